"""Pins for the oracle's small math: exp, rotation, SH basis, cameras.

The oracle restates gs3d in float32; each check below compares it with an
independent statement (NumPy/SciPy/float64 Torch autograd), never with a
retyped copy of the oracle's own formula.
"""

import math

import numpy as np
import pytest
import scipy.special
import torch

import torch_ref


def test_exp_accuracy(oracle_lib):
    # gs_expf must be within 3 ulp of exp on the range blending uses and
    # exact at 0 (alpha of a Gaussian at its own centre equals its opacity).
    x = np.concatenate([np.linspace(-86.0, 0.0, 200_001, dtype=np.float32),
                        -np.logspace(-8, 1.9, 5000).astype(np.float32)])
    got = oracle_lib.expf_array(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    err = np.abs(got - ref) / ulp
    assert err.max() <= 3.0, err.max()
    assert oracle_lib.expf(0.0) == 1.0
    assert oracle_lib.expf(-87.0) == 0.0
    # Monotone non-increasing as x decreases (threshold decisions stay ordered).
    xs = np.sort(x)
    ys = oracle_lib.expf_array(xs)
    assert np.all(np.diff(ys) >= 0)


def test_glm_rotation_is_transposed_standard_rotation(oracle_lib):
    rng = np.random.default_rng(0)
    for _ in range(200):
        q = rng.normal(size=4)
        q /= np.linalg.norm(q)
        R = oracle_lib.glm_rotation(q.astype(np.float32)).astype(np.float64)
        R_std = torch_ref.quat_to_rot(torch.tensor(q)).numpy()
        np.testing.assert_allclose(R, R_std.T, atol=2e-7)
    # Identity quaternion gives exactly the identity.
    np.testing.assert_array_equal(oracle_lib.glm_rotation([1, 0, 0, 0]), np.eye(3, dtype=np.float32))


def _real_sh_scipy(l, m, u):
    """Real spherical harmonics from SciPy's complex Y_l^m, in the sign
    convention of the 3DGS basis (checked against SH constants)."""
    x, y, z = u
    theta = math.acos(max(-1.0, min(1.0, z)))
    phi = math.atan2(y, x)
    if m == 0:
        return scipy.special.sph_harm_y(l, 0, theta, phi).real
    Y = scipy.special.sph_harm_y(l, abs(m), theta, phi)
    if m > 0:
        return math.sqrt(2) * (-1) ** m * Y.real
    return math.sqrt(2) * (-1) ** m * Y.imag


# 3DGS index k -> (l, m, sign): its basis equals sign * real Y_l^m.
_SH_INDEX = [(0, 0, 1), (1, -1, 1), (1, 0, 1), (1, 1, 1),
             (2, -2, 1), (2, -1, 1), (2, 0, 1), (2, 1, 1), (2, 2, 1),
             (3, -3, 1), (3, -2, 1), (3, -1, 1), (3, 0, 1), (3, 1, 1), (3, 2, 1), (3, 3, 1)]


def test_sh_basis_matches_scipy_real_harmonics(oracle_lib):
    # Each 3DGS basis function must equal a real spherical harmonic up to one
    # fixed sign per index (the 3DGS convention differs from SciPy's
    # Condon-Shortley phase for some m); a wrong constant, variable or sign
    # inside a polynomial breaks the equality or the sign consistency.
    rng = np.random.default_rng(1)
    signs = {}
    for _ in range(50):
        u = rng.normal(size=3)
        u /= np.linalg.norm(u)
        for k, (l, m, _) in enumerate(_SH_INDEX):
            ours = oracle_lib.sh_basis(u.astype(np.float32), k)
            ref = _real_sh_scipy(l, m, u)
            if abs(ref) < 1e-3:
                continue
            sign = 1.0 if ours * ref > 0 else -1.0
            signs.setdefault(k, sign)
            assert signs[k] == sign, (k, ours, ref)
            assert abs(ours - sign * ref) < 2e-6, (k, ours, ref)
    assert len(signs) == 16


def test_sh_basis_gradient_matches_autograd(oracle_lib):
    rng = np.random.default_rng(2)
    for _ in range(20):
        u = rng.normal(size=3)
        u /= np.linalg.norm(u)
        for k in range(16):
            coeffs = torch.zeros((1, 16, 3), dtype=torch.float64)
            coeffs[0, k, 0] = 1.0
            # Autograd of the textbook basis w.r.t. the (unit) direction.
            d = torch.tensor(u[None], requires_grad=True)
            x, y, z = d[0]
            val = _basis_torch(k, x, y, z)
            (g,) = torch.autograd.grad(val, d)
            ours = oracle_lib.sh_basis_grad(u.astype(np.float32), k)
            np.testing.assert_allclose(ours, g[0].numpy(), atol=2e-6, rtol=1e-5)


def _basis_torch(k, x, y, z):
    c1 = torch_ref.SH_C["c1"]
    c2, c3 = torch_ref.SH_C["c2"], torch_ref.SH_C["c3"]
    xx, yy, zz = x * x, y * y, z * z
    table = [
        lambda: torch_ref.SH_C["c0"] + 0 * x, lambda: -c1 * y, lambda: c1 * z, lambda: -c1 * x,
        lambda: c2[0] * x * y, lambda: c2[1] * y * z, lambda: c2[2] * (2 * zz - xx - yy),
        lambda: c2[3] * x * z, lambda: c2[4] * (xx - yy),
        lambda: c3[0] * y * (3 * xx - yy), lambda: c3[1] * x * y * z, lambda: c3[2] * y * (4 * zz - xx - yy),
        lambda: c3[3] * z * (2 * zz - 3 * xx - 3 * yy), lambda: c3[4] * x * (4 * zz - xx - yy),
        lambda: c3[5] * z * (xx - yy), lambda: c3[6] * x * (xx - 3 * yy),
    ]
    return table[k]()


def test_sh_forward_and_backward_against_torch(oracle_lib):
    rng = np.random.default_rng(3)
    n = 300
    for degree in range(4):
        coeffs = rng.normal(scale=0.4, size=(n, 16, 3)).astype(np.float32)
        dirs = rng.normal(size=(n, 3)).astype(np.float32)
        radii = (rng.random(n) > 0.2).astype(np.int32) * 3
        colors, active = oracle_lib.sh_fwd(coeffs, dirs, degree, radii)
        c64 = torch.tensor(coeffs, dtype=torch.float64, requires_grad=True)
        d64 = torch.tensor(dirs, dtype=torch.float64, requires_grad=True)
        ref = torch_ref.sh_colors(c64, d64, degree)
        vis = torch.tensor(radii > 0)
        ref = torch.where(vis[:, None], ref, torch.zeros_like(ref))
        np.testing.assert_allclose(colors, ref.detach().numpy(), atol=2e-6, rtol=1e-5)
        if degree == 0:
            # Closed form of SH0: max(C0*c + 0.5, 0) on visible rows.
            closed = np.maximum(np.float32(0.28209479177387814) * coeffs[:, 0] + np.float32(0.5), 0)
            np.testing.assert_array_equal(colors[radii > 0], closed[radii > 0])
        up = rng.normal(size=(n, 3)).astype(np.float32)
        gco, gdir = oracle_lib.sh_bwd(coeffs, dirs, degree, active, up, radii)
        # Reference gradient: clamp mask handled by autograd of clamp_min.
        (rc, rd) = torch.autograd.grad((ref * torch.tensor(up, dtype=torch.float64)).sum(), (c64, d64),
                                       allow_unused=True)
        np.testing.assert_allclose(gco, rc.numpy(), atol=5e-6, rtol=1e-4)
        if degree > 0:
            np.testing.assert_allclose(gdir, rd.numpy(), atol=5e-6, rtol=1e-4)
        assert np.all(gco[:, (degree + 1) ** 2:] == 0)


def test_camera_prepare_closed_form_and_errors(oracle_lib):
    rng = np.random.default_rng(4)
    views, Ks = [], []
    for _ in range(6):
        q = rng.normal(size=4)
        q /= np.linalg.norm(q)
        R = torch_ref.quat_to_rot(torch.tensor(q)).numpy()
        V = np.eye(4)
        V[:3, :3] = R
        V[:3, 3] = rng.normal(size=3)
        views.append(V.astype(np.float32))
        Ks.append(np.array([[500 + 100 * rng.random(), 0, 320 + rng.random()],
                            [0, 480 + 50 * rng.random(), 240 + rng.random()], [0, 0, 1]], np.float32))
    views, Ks = np.stack(views), np.stack(Ks)
    W, H = 640, 480
    full, inverse, centers, errors = oracle_lib.camera_prepare(views, Ks, W, H, True)
    assert np.all(errors == 0)
    f32 = np.float32
    for i in range(len(views)):
        K, V = Ks[i], views[i]
        px = f32(f32(2.0) * K[0, 0]) / f32(W)
        py = f32(f32(2.0) * K[1, 1]) / f32(H)
        cx = f32(f32(f32(2.0) * K[0, 2]) / f32(W)) - f32(1.0)
        cy = f32(f32(f32(2.0) * K[1, 2]) / f32(H)) - f32(1.0)
        expect = np.stack([px * V[0] + cx * V[2], py * V[1] + cy * V[2], V[2], V[2]])
        np.testing.assert_array_equal(full[i], expect.astype(np.float32))
        np.testing.assert_allclose(inverse[i], np.linalg.inv(V.astype(np.float64)), atol=1e-5)
        np.testing.assert_allclose(centers[i], torch_ref.look_at_rigid_inverse_center(
            torch.tensor(V, dtype=torch.float64)).numpy(), atol=1e-5)
    bad = Ks.copy()
    bad[0, 0, 0] = -1.0          # fx <= 0 -> 2
    bad[1, 0, 1] = 0.5           # skew -> 1
    bad[2, 1, 2] = np.nan        # non-finite -> 2
    bad[3, 2, 2] = 2.0           # not pinhole -> 1
    _, _, _, err = oracle_lib.camera_prepare(views, bad, W, H, True)
    assert list(err) == [2, 1, 2, 1, 0, 0]
    singular = views.copy()
    singular[4, 2] = singular[4, 1]
    _, _, _, err = oracle_lib.camera_prepare(singular, Ks, W, H, True)
    assert err[4] == 3 and err[0] == 0
    _, _, _, err = oracle_lib.camera_prepare(singular, Ks, W, H, False)
    assert err[4] == 0


def test_camera_backward_matches_autograd(oracle_lib):
    rng = np.random.default_rng(5)
    c = 3
    views = np.tile(np.eye(4, dtype=np.float32), (c, 1, 1))
    views[:, :3, 3] = rng.normal(size=(c, 3))
    views[:, :3, :3] += 0.1 * rng.normal(size=(c, 3, 3))
    Ks = np.stack([np.array([[700, 0, 300], [0, 650, 200], [0, 0, 1]], np.float32)] * c)
    W, H = 640, 480
    full, inverse, centers, err = oracle_lib.camera_prepare(views, Ks, W, H, True)
    g_full = rng.normal(size=(c, 4, 4)).astype(np.float32)
    g_cent = rng.normal(size=(c, 3)).astype(np.float32)
    ours = oracle_lib.camera_backward(Ks, g_full, W, H, inverse, g_cent)
    V = torch.tensor(views, dtype=torch.float64, requires_grad=True)
    K = torch.tensor(Ks, dtype=torch.float64)
    px = 2 * K[:, 0, 0] / W
    py = 2 * K[:, 1, 1] / H
    cx = 2 * K[:, 0, 2] / W - 1
    cy = 2 * K[:, 1, 2] / H - 1
    P = torch.stack([px[:, None] * V[:, 0] + cx[:, None] * V[:, 2],
                     py[:, None] * V[:, 1] + cy[:, None] * V[:, 2], V[:, 2], V[:, 2]], 1)
    cen = torch.linalg.inv(V)[:, :3, 3]
    loss = (P * torch.tensor(g_full, dtype=torch.float64)).sum() + (cen * torch.tensor(g_cent, dtype=torch.float64)).sum()
    (gv,) = torch.autograd.grad(loss, V)
    np.testing.assert_allclose(ours, gv.numpy(), rtol=1e-4, atol=1e-4)


def test_logf_is_the_rounded_float64_log(oracle_lib):
    # The footprint's natural log (splatting/intersections.py:68, wp.log):
    # a double computation rounded once, so it is the float32 rounding of
    # the exact log except where that rounding is a near tie; always within
    # one float32 ulp.  Covers the alpha levels 255*o for o in (1/255, 1]
    # densely and the rest of the positive float range sparsely.
    rng = np.random.default_rng(5)
    levels = np.concatenate([np.linspace(1.0, 255.0, 20001), rng.uniform(1.0, 255.0, 20000),
                             10.0 ** rng.uniform(-30, 30, 20000)]).astype(np.float32)
    got = np.array([oracle_lib.logf(float(x)) for x in levels], np.float32)
    exact = np.log(levels.astype(np.float64))
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - exact) <= ulp)
    assert np.mean(got == exact.astype(np.float32)) > 0.9999
    assert oracle_lib.logf(1.0) == 0.0
