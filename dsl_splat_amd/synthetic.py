"""Seeded synthetic scenes for the five rasterizer workloads.

Every tensor is drawn on the CPU in float32 from one torch.Generator seeded
with ``seed``, in the order listed for each workload, then moved to
``device``.  Cameras use the OpenCV look-at convention: z = normalize(target -
eye), x = normalize(z x (0,1,0)), y = z x x, R = [x; y; z], t = -R eye.

Workloads (``name``):
  small     N=10k, 256x256, identity pose, fx=fy=256, RGB features U[0,1]
  sh3_720p  N=500k, 1280x720, eye (0,0,-4), fx=fy=1000, SH3, absgrad
  sh3_1080p_4view  N=3M, 1920x1080, 4 cameras on a radius-5 ring, 64 clusters,
            SH3 (the headline workload)
  feat32    N=1M, 1600x1200, 32 feature channels + camera-z extra channel
  pose_fanout  N=2M, 1920x1080, SH3, 5% large Gaussians, pose gradients
``n``/``width``/``height`` override the sizes (used for small parity cases).
"""

from dataclasses import dataclass, field
import math

import torch


@dataclass
class Scene:
    name: str
    means: torch.Tensor
    quats: torch.Tensor
    scales: torch.Tensor
    opacities: torch.Tensor
    viewmats: torch.Tensor
    Ks: torch.Tensor
    width: int
    height: int
    features: torch.Tensor | None = None
    sh_coeffs: torch.Tensor | None = None
    sh_degree: int | None = None
    extra_features: torch.Tensor | None = None
    absgrad: bool = False
    pose_grad: bool = False
    loss_weights: torch.Tensor | None = None
    kwargs: dict = field(default_factory=dict)

    def to(self, device) -> "Scene":
        for name in ("means", "quats", "scales", "opacities", "viewmats", "Ks", "features",
                     "sh_coeffs", "extra_features", "loss_weights"):
            value = getattr(self, name)
            if value is not None:
                setattr(self, name, value.to(device))
        return self


def look_at(eye, target=(0.0, 0.0, 0.0)) -> torch.Tensor:
    eye = torch.tensor(eye, dtype=torch.float64)
    target = torch.tensor(target, dtype=torch.float64)
    z = target - eye
    z = z / z.norm()
    x = torch.linalg.cross(z, torch.tensor([0.0, 1.0, 0.0], dtype=torch.float64))
    x = x / x.norm()
    y = torch.linalg.cross(z, x)
    R = torch.stack([x, y, z])
    view = torch.eye(4, dtype=torch.float64)
    view[:3, :3] = R
    view[:3, 3] = -R @ eye
    return view.float()


def intrinsics(f, width, height) -> torch.Tensor:
    return torch.tensor([[f, 0.0, width / 2.0], [0.0, f, height / 2.0], [0.0, 0.0, 1.0]],
                        dtype=torch.float32)


def _uniform(g, shape, lo, hi):
    return torch.rand(shape, generator=g) * (hi - lo) + lo


def _ball(g, n, radius):
    d = torch.randn((n, 3), generator=g)
    d = d / d.norm(dim=-1, keepdim=True)
    r = radius * torch.rand((n, 1), generator=g) ** (1.0 / 3.0)
    return d * r


def _quats(g, n):
    q = torch.randn((n, 4), generator=g)
    return q / q.norm(dim=-1, keepdim=True)


def _sh3(g, n):
    sh = torch.empty((n, 16, 3))
    sh[:, :1] = torch.randn((n, 1, 3), generator=g) * 0.5
    sh[:, 1:] = torch.randn((n, 15, 3), generator=g) * 0.05
    return sh


def make_scene(name: str, *, n: int | None = None, width: int | None = None,
               height: int | None = None, seed: int = 0, device="cpu") -> Scene:
    g = torch.Generator("cpu").manual_seed(seed)
    if name == "small":
        n = n or 10_000
        width, height = width or 256, height or 256
        means = _uniform(g, (n, 3), -1.0, 1.0)
        means[:, 2] += 4.0
        scales = torch.exp(_uniform(g, (n, 3), -4.5, -2.5))
        quats = _quats(g, n)
        opac = torch.sigmoid(torch.randn(n, generator=g))
        feats = torch.rand((n, 3), generator=g)
        view = torch.eye(4)[None]
        K = torch.tensor([[256.0 * width / 256, 0, width / 2], [0, 256.0 * height / 256, height / 2],
                          [0, 0, 1]])[None]
        scene = Scene(name, means, quats, scales, opac, view, K, width, height, features=feats)
        channels = 4
    elif name == "sh3_720p":
        n = n or 500_000
        width, height = width or 1280, height or 720
        means = _ball(g, n, 1.5)
        scales = torch.exp(_uniform(g, (n, 3), -5.0, -3.0))
        quats = _quats(g, n)
        opac = torch.sigmoid(torch.randn(n, generator=g))
        sh = _sh3(g, n)
        f = 1000.0 * width / 1280
        scene = Scene(name, means, quats, scales, opac, look_at((0.0, 0.0, -4.0))[None],
                      intrinsics(f, width, height)[None], width, height, sh_coeffs=sh,
                      sh_degree=3, absgrad=True)
        channels = 4
    elif name == "sh3_1080p_4view":
        n = n or 3_000_000
        width, height = width or 1920, height or 1080
        centres = _uniform(g, (64, 3), -2.0, 2.0)
        assign = torch.randint(0, 64, (n,), generator=g)
        means = centres[assign] + 0.3 * torch.randn((n, 3), generator=g)
        scales = torch.exp(_uniform(g, (n, 3), -5.5, -3.0))
        quats = _quats(g, n)
        opac = torch.sigmoid(1.5 * torch.randn(n, generator=g))
        sh = _sh3(g, n)
        f = 1400.0 * width / 1920
        views = torch.stack([look_at((5.0 * math.sin(math.radians(a)), 0.0, -5.0 * math.cos(math.radians(a))))
                             for a in (0.0, 90.0, 180.0, 270.0)])
        Ks = intrinsics(f, width, height)[None].repeat(4, 1, 1)
        scene = Scene(name, means, quats, scales, opac, views, Ks, width, height, sh_coeffs=sh, sh_degree=3)
        channels = 4
    elif name == "feat32":
        n = n or 1_000_000
        width, height = width or 1600, height or 1200
        means = _ball(g, n, 1.5)
        scales = torch.exp(_uniform(g, (n, 3), -5.0, -3.0))
        quats = _quats(g, n)
        opac = torch.sigmoid(torch.randn(n, generator=g))
        feats = torch.randn((n, 32), generator=g)
        view = look_at((0.0, 0.0, -4.0))[None]
        f = 1200.0 * width / 1600
        # Camera-space z of each mean as the extra (expected-depth) channel.
        z = (means @ view[0, 2, :3] + view[0, 2, 3])[None, :, None].contiguous()
        scene = Scene(name, means, quats, scales, opac, view, intrinsics(f, width, height)[None], width,
                      height, features=feats, extra_features=z)
        channels = 34
    elif name == "pose_fanout":
        n = n or 2_000_000
        width, height = width or 1920, height or 1080
        means = _uniform(g, (n, 3), -2.0, 2.0)
        perm = torch.randperm(n, generator=g)
        large = perm[: max(1, n // 20)]
        log_scales = _uniform(g, (n, 3), -7.0, -5.0)
        log_scales[large] = _uniform(g, (len(large), 3), -1.0, 0.0)
        scales = torch.exp(log_scales)
        quats = _quats(g, n)
        opac = torch.sigmoid(torch.randn(n, generator=g))
        sh = _sh3(g, n)
        f = 1400.0 * width / 1920
        scene = Scene(name, means, quats, scales, opac, look_at((0.0, 0.0, -5.0))[None],
                      intrinsics(f, width, height)[None], width, height, sh_coeffs=sh, sh_degree=3,
                      absgrad=True, pose_grad=True)
        channels = 4
    else:
        raise ValueError(f"unknown scene {name!r}")
    cameras = scene.viewmats.shape[0]
    rgb = channels - 1
    scene.loss_weights = torch.randn((cameras, height, width, rgb + 1), generator=g)
    return scene.to(device)


WORKLOADS = ("small", "sh3_720p", "sh3_1080p_4view", "feat32", "pose_fanout")
