"""DistortedPerspectiveCamera: reference src/xsimgs/cameras/ext/distorted_perspective.py with
cameras/torch/distorted_perspective.py and distortion_utils.py (OpenCV rational radial + tangential
model, coefficients k1, k2, p1, p2, k3, k4, k5, k6, on normalised intrinsics [fx/W, fy/H, cx/W, cy/H])."""
import torch

from .._C import DistortedPerspectiveCamera as CDistortedPerspectiveCamera
from .ext_camera import CameraPose
from .perspective import PerspectiveCamera


def max_valid_radius(normalized_intrinsics: torch.Tensor, distortion: torch.Tensor, margin: float = 1.5,
                     search_limit: float = 16.0, num_samples: int = 8192) -> torch.Tensor:
    """Largest camera-space radius r = |xy| / z the calibration is evaluated at (distortion_utils.py:
    max_valid_radius): the smaller of the radius where the radial map rho(r) = r * scale(r) stops
    increasing (the lens folds) and `margin` times the radius of the farthest image corner, both read
    off `num_samples` radii in [0, search_limit]. Returns [..., 1] like `distortion`."""
    dist = distortion.reshape(-1, 8)
    intr = normalized_intrinsics.reshape(-1, 4).to(dist)
    r = torch.linspace(0.0, search_limit, num_samples, device=dist.device, dtype=dist.dtype)
    r2 = r * r
    k1, k2, _, _, k3, k4, k5, k6 = (dist[:, i:i + 1] for i in range(8))
    rho = r * (1.0 + r2 * (k1 + r2 * (k2 + r2 * k3))) / (1.0 + r2 * (k4 + r2 * (k5 + r2 * k6)))
    falls = rho[:, 1:] < rho[:, :-1]
    first_fall = torch.where(falls.any(-1), falls.to(torch.int64).argmax(-1),
                             torch.full_like(falls[:, 0], num_samples - 1, dtype=torch.int64))
    r_fold = r[first_fall]
    corners = torch.tensor([[0.0, 0.0], [1.0, 0.0], [0.0, 1.0], [1.0, 1.0]], device=dist.device, dtype=dist.dtype)
    rho_corner = ((corners[None] - intr[:, None, 2:]) / intr[:, None, :2]).norm(dim=-1).amax(-1)
    rising = torch.cummax(rho, dim=-1).values.contiguous()
    idx = torch.searchsorted(rising, rho_corner[:, None]).squeeze(-1).clamp(max=num_samples - 1)
    r_corner = r[idx]
    return torch.minimum(r_fold, margin * r_corner).reshape(*distortion.shape[:-1], 1)


class DistortedPerspectiveCamera(PerspectiveCamera):
    ext_cls = CDistortedPerspectiveCamera
    undistorted_cls = PerspectiveCamera
    max_radius_margin: float = 1.5

    def __init__(self, pose: CameraPose, normalized_intrinsics: torch.Tensor, distortion: torch.Tensor):
        super().__init__(pose, normalized_intrinsics)
        self.distortion = torch.as_tensor(distortion, dtype=torch.float32, device=pose.q.device).contiguous()
        assert self.distortion.shape[-1] == 8, \
            "Distortion coefficients must be of [..., 8] shape: k1, k2, p1, p2, k3, k4, k5, k6"
        self._max_radius = None

    @property
    def max_radius(self) -> torch.Tensor:
        """Radius bound of this calibration ([1]), derived from the coefficients and intrinsics and cached."""
        if self._max_radius is None:
            self._max_radius = max_valid_radius(self.normalized_intrinsics.detach(), self.distortion.detach(),
                                                margin=self.max_radius_margin)
        return self._max_radius

    @property
    def _pack_data(self):
        # max_radius goes in squared: the projection compares it with r^2 (distorted_perspective.py:19-21)
        return super()._pack_data + [self.distortion.view(8).contiguous(),
                                     self.max_radius.reshape(1).square().contiguous()]

    def undistort(self) -> PerspectiveCamera:
        return self.undistorted_cls(self.pose, self.normalized_intrinsics)
