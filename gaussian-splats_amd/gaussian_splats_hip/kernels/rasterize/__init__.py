"""HIP (gfx950) rasterizer stages and the ``gaussian_splats_hip::rasterize`` op."""

from .composite import composite
from .composite_bwd import composite_bwd
from .interface import rasterize
from .intersections import (
    bin_gaussians,
    bin_tiles,
    depth_key_range,
    emit_intersections,
    emit_tiles,
    sort_intersections,
    sort_tiles,
)
from .project import pack_records, project_and_count
from .project_bwd import project_bwd
from .views import rasterize_views

__all__ = [
    "bin_gaussians",
    "bin_tiles",
    "composite",
    "composite_bwd",
    "depth_key_range",
    "emit_intersections",
    "emit_tiles",
    "pack_records",
    "project_and_count",
    "project_bwd",
    "rasterize",
    "rasterize_views",
    "sort_intersections",
    "sort_tiles",
]
