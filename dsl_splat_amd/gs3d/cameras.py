"""Camera preparation and the 3DGS view configuration with its tile mode
(gs3d/cameras.py:1-38 of the reference)."""

from dataclasses import dataclass

from ..cameras import PinholeCamera
from ..splatting.cameras import (  # noqa: F401  (re-exports)
    ViewConfig as _ViewConfig,
    _PrepareCameras,
    prepare_camera as _prepare_camera,
    prepare_cameras,
    prepare_cameras_with_centers,
)


@dataclass(frozen=True, slots=True)
class ViewConfig(_ViewConfig):
    tile_mode: str = "radius"


def prepare_camera(camera: PinholeCamera, radius_clip: float, bindings=None):
    view, projection, intrinsics, config = _prepare_camera(camera, radius_clip, bindings)
    return view, projection, intrinsics, ViewConfig(config.width, config.height, config.near, config.far,
                                                    config.radius_clip)
