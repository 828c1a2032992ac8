from gaussian_splatting.scene.camera import camera
from gaussian_splatting.scene.gaussian import gaussian

__all__ = ["camera", "gaussian"]
