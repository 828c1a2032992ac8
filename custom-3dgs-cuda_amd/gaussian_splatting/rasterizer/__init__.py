from gaussian_splatting.rasterizer.bands import band_rows, band_views, rasterize_bands
from gaussian_splatting.rasterizer.rasterize import RasterizeFunction, rasterize

__all__ = ["RasterizeFunction", "rasterize", "rasterize_bands", "band_rows", "band_views"]
