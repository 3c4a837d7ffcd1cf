"""PerspectiveCamera: reference src/xsimgs/cameras/ext/perspective.py and
cameras/torch/perspective.py (normalized intrinsics [fx/W, fy/H, cx/W, cy/H])."""
import torch

from .._C import PerspectiveCamera as CPerspectiveCamera
from .ext_camera import CameraPose, FusedRSCamera


class PerspectiveCamera(FusedRSCamera):
    ext_cls = CPerspectiveCamera

    def __init__(self, pose: CameraPose, normalized_intrinsics: torch.Tensor):
        super().__init__(pose)
        self.normalized_intrinsics = torch.as_tensor(normalized_intrinsics, dtype=torch.float32,
                                                     device=pose.q.device).reshape(4).contiguous()

    @staticmethod
    def intrinsics_from_sized(fx, fy, cx, cy, width, height) -> torch.Tensor:
        return torch.tensor([fx / width, fy / height, cx / width, cy / height], dtype=torch.float32)

    @property
    def _pack_data(self):
        return super()._pack_data + [self.normalized_intrinsics.view(4).contiguous()]
