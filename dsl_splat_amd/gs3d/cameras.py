"""Camera preparation for the 3DGS entry points, with the view
configuration extended by the tile mode (the role of gs3d/cameras.py:1-38 of
the reference)."""

from dataclasses import dataclass

from ..cameras import PinholeCamera
from ..splatting import cameras as _shared
from ..splatting.cameras import prepare_cameras, prepare_cameras_with_centers  # noqa: F401  (re-exports)


@dataclass(frozen=True, slots=True)
class ViewConfig(_shared.ViewConfig):
    tile_mode: str = "radius"  # "radius", "snugbox" or "accutile"


def prepare_camera(camera: PinholeCamera, radius_clip: float, bindings=None):
    """splatting.cameras.prepare_camera with a 3DGS ViewConfig (tile mode "radius")."""
    view, projection, intrinsics, base = _shared.prepare_camera(camera, radius_clip, bindings)
    return view, projection, intrinsics, ViewConfig(base.width, base.height, base.near, base.far, base.radius_clip)
