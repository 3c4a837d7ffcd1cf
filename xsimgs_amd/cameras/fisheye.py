"""FisheyeCamera: reference src/xsimgs/cameras/ext/fisheye.py with cameras/torch/fisheye.py (OpenCV
fisheye / Kannala-Brandt model theta_d = theta (1 + k1 theta^2 + k2 theta^4 + k3 theta^6 + k4 theta^8)
on normalised intrinsics [fx/W, fy/H, cx/W, cy/H])."""
import torch

from .._C import OpenCVFisheyeCamera as CFisheyeCamera
from .ext_camera import CameraPose
from .perspective import PerspectiveCamera


class FisheyeCamera(PerspectiveCamera):
    ext_cls = CFisheyeCamera

    def __init__(self, pose: CameraPose, normalized_intrinsics: torch.Tensor, distortion: torch.Tensor):
        super().__init__(pose, normalized_intrinsics)
        self.distortion = torch.as_tensor(distortion, dtype=torch.float32, device=pose.q.device).contiguous()
        assert self.distortion.shape[-1] == 4, "Distortion coefficients must be of [..., 4] shape: k1, k2, k3, k4"

    @property
    def _pack_data(self):
        return super()._pack_data + [self.distortion.view(4).contiguous()]
