"""Camera container; layouts of gaussian_splatting/scene/camera.py:3-38."""

import torch as t


class camera:
    """N pinhole cameras: world-to-camera R [N,3,3] and t [N,3], intrinsics [N,1]."""

    def __init__(self, N):
        self.N = N
        self.R = t.zeros(N, 3, 3, dtype=t.float32)
        self.t = t.zeros(N, 3, dtype=t.float32)
        self.fx = t.zeros(N, 1, dtype=t.float32)
        self.fy = t.zeros(N, 1, dtype=t.float32)
        self.cx = t.zeros(N, 1, dtype=t.float32)
        self.cy = t.zeros(N, 1, dtype=t.float32)

    def sample_camera_view(self):
        """One view dict per camera (the keys ``rasterize`` reads), with optional paths."""
        image_paths = getattr(self, "image_paths", [None] * self.N)
        image_names = getattr(self, "image_names", [None] * self.N)
        return [
            {
                "R": self.R[i],
                "T": self.t[i],
                "fx": self.fx[i],
                "fy": self.fy[i],
                "cx": self.cx[i],
                "cy": self.cy[i],
                "image_path": image_paths[i],
                "image_name": image_names[i],
            }
            for i in range(self.N)
        ]
