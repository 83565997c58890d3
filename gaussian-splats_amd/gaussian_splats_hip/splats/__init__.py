from .camera import Camera, PinholeCamera
from .rasterize import rasterize, rasterize_views
from .splats import GaussianSplat, ProjectedGaussianSplat
from .utils import SH_C0, quaternion_to_rotation_matrix, rgb_to_sh

__all__ = [
    "SH_C0",
    "Camera",
    "GaussianSplat",
    "PinholeCamera",
    "ProjectedGaussianSplat",
    "quaternion_to_rotation_matrix",
    "rasterize",
    "rasterize_views",
    "rgb_to_sh",
]
