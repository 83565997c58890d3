"""MI355X-native differentiable Gaussian-splat rasterizer.

The public API mirrors the ``gaussian_splats`` package of
VikaasVarma/gaussian-splats for the render path (under its own name, so that
both can be imported in one process): :class:`gaussian_splats_hip.splats.GaussianSplat`,
:class:`gaussian_splats_hip.splats.PinholeCamera` and
:func:`gaussian_splats_hip.splats.rasterize`, backed by hand-written gfx950 HIP
kernels behind the C ABI of ``include/gs_raster.h``.
"""

__version__ = "0.1.0"
