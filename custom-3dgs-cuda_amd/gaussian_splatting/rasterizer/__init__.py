from gaussian_splatting.rasterizer.rasterize import RasterizeFunction, rasterize

__all__ = ["RasterizeFunction", "rasterize"]
