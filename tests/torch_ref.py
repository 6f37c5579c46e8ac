"""Independent float64 Torch statement of the gs3d math, for pinning the oracle.

Written from the textbook EWA-splatting formulas (standard quaternion
rotation, Sigma = R S^2 R^T, J = d(proj)/d(cam), cov2 = J W Sigma W^T J^T),
not from the oracle's op sequence, so agreement with the oracle checks the
oracle's restatement rather than retyping it.  Autograd supplies reference
VJPs; the two conventions of the reference that are not exact derivatives
are reproduced explicitly:
  * saturated clamp components are detached (splatting/geometry.py:42-51);
  * the inverse-covariance VJP uses 1/(det^2 + 1e-7) instead of 1/det^2
    (splatting/geometry.py:61-71), via a custom autograd Function.
"""

import math

import torch

SH_C = dict(
    c0=0.28209479177387814, c1=0.4886025119029199, c2=(1.0925484305920792, -1.0925484305920792,
                                                         0.31539156525252005, -1.0925484305920792,
                                                         0.5462742152960396),
    c3=(-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154,
        -0.4570457994644658, 1.445305721320277, -0.5900435899266435),
)


def quat_to_rot(q):
    """Standard rotation matrix of a unit quaternion (w, x, y, z)."""
    w, x, y, z = q.unbind(-1)
    return torch.stack([
        torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1),
        torch.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], -1),
        torch.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1),
    ], -2)


class _RegularisedInverse(torch.autograd.Function):
    """(a,b,c) -> (c,-b,a)/det with the reference's regularised VJP."""

    @staticmethod
    def forward(ctx, cov):
        a, b, c = cov.unbind(-1)
        det = a * c - b * b
        ctx.save_for_backward(cov)
        return torch.stack([c / det, -b / det, a / det], -1)

    @staticmethod
    def backward(ctx, g):
        (cov,) = ctx.saved_tensors
        with torch.enable_grad():
            x = cov.detach().requires_grad_(True)
            a, b, c = x.unbind(-1)
            det = a * c - b * b
            y = torch.stack([c / det, -b / det, a / det], -1)
            (exact,) = torch.autograd.grad(y, x, g)
        a, b, c = cov.unbind(-1)
        det = a * c - b * b
        return exact * (det * det / (det * det + 1e-7))[..., None]


def project(means, quats, scales, opacities, view, K, width, height):
    """Projected centres (pixel, integer-centre convention), conic (a,b,c),
    opacity and camera depth of every Gaussian for one camera (no culling)."""
    fx, fy = K[0, 0], K[1, 1]
    R3, t3 = view[:3, :3], view[:3, 3]
    p = means @ R3.T + t3
    limx = 1.3 * width / (2 * fx)
    limy = 1.3 * height / (2 * fy)
    xr, yr = p[:, 0] / p[:, 2], p[:, 1] / p[:, 2]
    sat_x = (xr < -limx) | (xr > limx)
    sat_y = (yr < -limy) | (yr > limy)
    tx = torch.where(sat_x, (xr.clamp(-limx, limx) * p[:, 2]).detach(), p[:, 0])
    ty = torch.where(sat_y, (yr.clamp(-limy, limy) * p[:, 2]).detach(), p[:, 1])
    tz = p[:, 2]
    zero = torch.zeros_like(tz)
    J = torch.stack([
        torch.stack([fx / tz, zero, -fx * tx / tz ** 2], -1),
        torch.stack([zero, fy / tz, -fy * ty / tz ** 2], -1),
    ], -2)
    R = quat_to_rot(quats)
    S2 = torch.diag_embed(scales ** 2)
    sigma = R @ S2 @ R.transpose(-1, -2)
    T = J @ R3
    cov = T @ sigma @ T.transpose(-1, -2)
    cov3 = torch.stack([cov[:, 0, 0] + 0.3, cov[:, 0, 1], cov[:, 1, 1] + 0.3], -1)
    conic = _RegularisedInverse.apply(cov3)
    # Pixel centre from the full projection (== K-projection minus 0.5).
    cx = fx * p[:, 0] / p[:, 2] + K[0, 2] - 0.5
    cy = fy * p[:, 1] / p[:, 2] + K[1, 2] - 0.5
    centers = torch.stack([cx, cy], -1)
    return centers, conic, opacities, p[:, 2], cov3


def sh_colors(coeffs, dirs, degree):
    """Textbook real SH (the inputs.py:63-98 form), +0.5, clamped at 0."""
    d = dirs / dirs.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    x, y, z = d.unbind(-1)
    basis = [torch.full_like(x, SH_C["c0"])]
    if degree >= 1:
        c1 = SH_C["c1"]
        basis += [-c1 * y, c1 * z, -c1 * x]
    if degree >= 2:
        c = SH_C["c2"]
        xx, yy, zz = x * x, y * y, z * z
        basis += [c[0] * x * y, c[1] * y * z, c[2] * (2 * zz - xx - yy), c[3] * x * z, c[4] * (xx - yy)]
    if degree >= 3:
        c = SH_C["c3"]
        xx, yy, zz = x * x, y * y, z * z
        basis += [c[0] * y * (3 * xx - yy), c[1] * x * y * z, c[2] * y * (4 * zz - xx - yy),
                  c[3] * z * (2 * zz - 3 * xx - 3 * yy), c[4] * x * (4 * zz - xx - yy),
                  c[5] * z * (xx - yy), c[6] * x * (xx - 3 * yy)]
    w = torch.stack(basis, -1)
    return ((coeffs[:, : len(basis)] * w[..., None]).sum(-2) + 0.5).clamp_min(0)


def render(centers, conics, opacities, colors, order, width, height, background=None, radii=None):
    """Per-pixel front-to-back blend of the Gaussians listed in ``order``
    (already depth sorted), same rules as gs3d/render.py:85-117, vectorised
    over pixels.  With ``radii`` a Gaussian only reaches the pixels of the
    16x16 tiles its square rectangle covers (the binning of the reference).
    Returns image (H,W,D+1) with the alpha channel last, and T_final."""
    ys, xs = torch.meshgrid(torch.arange(height, dtype=centers.dtype),
                            torch.arange(width, dtype=centers.dtype), indexing="ij")
    D = colors.shape[-1]
    T = torch.ones((height, width), dtype=centers.dtype)
    color = torch.zeros((height, width, D + 1), dtype=centers.dtype)
    done = torch.zeros((height, width), dtype=torch.bool)
    feats = torch.cat([colors, torch.ones_like(colors[:, :1])], -1)
    for g in order:
        member = torch.ones((height, width), dtype=torch.bool)
        if radii is not None:
            x0, y0, x1, y1 = rect_tiles(centers[g].detach().float().tolist(), int(radii[g]), width, height)
            tx, ty = (xs // 16).long(), (ys // 16).long()
            member = (tx >= x0) & (tx < x1) & (ty >= y0) & (ty < y1)
        dx = centers[g, 0] - xs
        dy = centers[g, 1] - ys
        a, b, c = conics[g].unbind(-1)
        power = -0.5 * (a * dx * dx + c * dy * dy) - b * dx * dy
        alpha = torch.clamp(opacities[g] * torch.exp(power), max=0.99)
        ok = (power <= 0) & (alpha >= 1.0 / 255.0) & ~done & member
        next_t = T * (1 - alpha)
        stop = ok & (next_t < 1e-4)
        blend = ok & ~stop
        w = torch.where(blend, alpha * T, torch.zeros_like(T))
        color = color + w[..., None] * feats[g]
        T = torch.where(blend, next_t, T)
        done = done | stop
    if background is not None:
        bg = torch.cat([background, torch.zeros(1, dtype=background.dtype)])
        color = color + T[..., None] * bg
    return color, T


def rect_tiles(center, radius, width, height):
    """Tile rectangle of one Gaussian (CUDA getRect truncation) in Python."""
    gx, gy = (width + 15) // 16, (height + 15) // 16
    f32 = lambda v: float(torch.tensor(v, dtype=torch.float32))
    def tc(v, hi):
        return min(max(int(v), 0), hi)
    r = float(radius)
    x0 = tc(f32(f32(center[0] - r) / 16.0), gx)
    y0 = tc(f32(f32(center[1] - r) / 16.0), gy)
    x1 = tc(f32(f32(f32(f32(center[0] + r) + 16.0) - 1.0) / 16.0), gx)
    y1 = tc(f32(f32(f32(f32(center[1] + r) + 16.0) - 1.0) / 16.0), gy)
    return x0, y0, x1, y1


def look_at_rigid_inverse_center(view):
    """Camera centre of a rigid world->camera matrix: -R^T t."""
    R, t = view[:3, :3], view[:3, 3]
    return -(R.T @ t)


def radius_of(cov3):
    a, b, c = cov3
    det = a * c - b * b
    mid = 0.5 * (a + c)
    lam = mid + math.sqrt(max(0.1, mid * mid - det))
    return 3.0 * math.sqrt(lam)
