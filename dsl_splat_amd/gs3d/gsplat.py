"""gsplat's ``rasterization`` signature over the original-3DGS HIP pipeline
(the contract of gs3d/gsplat.py:15-194 of the reference).

Only what original 3DGS defines is accepted -- pinhole cameras, global
shutter, RGB/feature rendering with the fixed 0.3 dilation on 16-pixel tiles;
every other option raises NotImplementedError before any work, in the
reference's order and with its messages, and size, clip and SH options raise
ValueError.  gsplat's defaults are kept (near 0.01, far 1e10, packed=True);
``colors`` are SH coefficients exactly when ``sh_degree`` is given.  means2d
keeps CUDA's integer-centre raster coordinates.
"""

from numbers import Integral
from typing import Any, Literal, Sequence

from torch import Tensor

from .api import rasterize
from ..cameras import validate_camera_options
from ..inputs import RenderMode
from ..statistics import StatisticsRequest

# Options original 3DGS does not have: flags that must stay False, inputs that
# must stay None.
_FLAGS = ("sparse_grad", "distributed", "segmented", "with_ut")
_ABSENT = ("covars", "radial_coeffs", "tangential_coeffs", "thin_prism_coeffs", "ftheta_coeffs", "viewmats_rs",
           "extra_signals_sh_degree")


def _positive_int(v) -> bool:
    return isinstance(v, Integral) and not isinstance(v, bool) and v > 0


def _reject(options: dict[str, Any]) -> None:
    for flag in _FLAGS:
        if options[flag]:
            raise NotImplementedError(f"3DGS/HIP gsplat adapter does not support {flag}=True")
    for name in _ABSENT:
        if options[name] is not None:
            raise NotImplementedError(f"3DGS/HIP gsplat adapter does not support {name}")
    shutter = options["rolling_shutter"]
    shutter = getattr(shutter, "name", shutter)
    requirements = (
        (shutter in (None, 0, "GLOBAL", "global"), "only global shutter is supported"),
        (options["camera_model"] == "pinhole", "only pinhole cameras are supported"),
        (options["with_eval3d"] is not True,
         "original 3DGS uses projected 2D conics; with_eval3d=True is unsupported"),
        (options["eps2d"] == 0.3, "original 3DGS currently has fixed eps2d=0.3"),
        (options["tile_size"] in (None, 16), "original 3DGS currently requires tile_size=16"),
        (options["render_mode"] == "RGB",
         "3DGS/HIP supports render_mode='RGB' for RGB or arbitrary features; depth rendering is not implemented"),
        (options["rasterize_mode"] == "classic", "original 3DGS supports rasterize_mode='classic' only"),
    )
    for satisfied, message in requirements:
        if not satisfied:
            raise NotImplementedError(message)
    if not all(_positive_int(options[k]) for k in ("width", "height", "channel_chunk")):
        raise ValueError("width, height and channel_chunk must be positive integers")
    validate_camera_options(options["width"], options["height"], options["near_plane"], options["far_plane"],
                            options["radius_clip"])
    sh_degree = options["sh_degree"]
    if sh_degree is not None and (isinstance(sh_degree, bool) or not isinstance(sh_degree, Integral)
                                  or not 0 <= sh_degree <= 3):
        raise ValueError("sh_degree must be None or an integer in [0,3]")


def rasterization(
    means: Tensor,
    quats: Tensor,
    scales: Tensor,
    opacities: Tensor,
    colors: Tensor | None,
    viewmats: Tensor,
    Ks: Tensor,
    width: int,
    height: int,
    near_plane: float = 0.01,
    far_plane: float = 10000000000.0,
    radius_clip: float = 0.0,
    eps2d: float = 0.3,
    sh_degree: int | None = None,
    packed: bool = True,
    tile_size: int | None = 16,
    backgrounds: Tensor | None = None,
    render_mode: RenderMode = "RGB",
    sparse_grad: bool = False,
    absgrad: bool = False,
    rasterize_mode: Literal["classic", "antialiased"] = "classic",
    channel_chunk: int = 32,
    distributed: bool = False,
    camera_model: str = "pinhole",
    segmented: bool = False,
    covars: Tensor | None = None,
    with_ut: bool = False,
    with_eval3d: bool | None = None,
    radial_coeffs: Tensor | None = None,
    tangential_coeffs: Tensor | None = None,
    thin_prism_coeffs: Tensor | None = None,
    ftheta_coeffs: object | None = None,
    rolling_shutter: object | None = None,
    viewmats_rs: Tensor | None = None,
    *,
    extra_signals: Tensor | None = None,
    extra_signals_sh_degree: int | None = None,
    statistics: Sequence[StatisticsRequest] = (),
    tile_mode: str = "radius",
) -> tuple[Tensor, Tensor, dict[str, Any]]:
    """(features, alpha, meta) of gs3d.rasterize under gsplat's names;
    requested statistics also appear as meta["statistics"]."""
    _reject(dict(locals()))
    result = rasterize(
        means, quats, scales, opacities, viewmats, Ks, width, height,
        features=None if sh_degree is not None else colors,
        sh_coeffs=colors if sh_degree is not None else None,
        sh_degree=sh_degree, backgrounds=backgrounds, extra_features=extra_signals, near_plane=near_plane,
        far_plane=far_plane, radius_clip=radius_clip, packed=packed, absgrad=absgrad, statistics=statistics,
        tile_mode=tile_mode,
    )
    if statistics:
        result.meta["statistics"] = result.statistics
    return result.features, result.alpha, result.meta


__all__ = ["rasterization"]
