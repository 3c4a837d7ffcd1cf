"""SphericalCamera: reference src/xsimgs/cameras/ext/spherical.py:21-67 (limits =
[phi_min, phi_range, theta_min, theta_range], cameras/torch/spherical.py:117-152)."""
import torch

from .._C import SphericalCamera as CSphericalCamera, isect_spherical_tiles
from .ext_camera import CameraPose, FusedRSCamera


class SphericalCamera(FusedRSCamera):
    ext_cls = CSphericalCamera

    def __init__(self, pose: CameraPose, limits: torch.Tensor = None):
        super().__init__(pose)
        if limits is None:
            limits = torch.tensor([0.0, 2 * torch.pi, -torch.pi / 2.0, torch.pi])
        limits = torch.as_tensor(limits, dtype=torch.float32, device=pose.q.device).reshape(4).contiguous()
        assert float(limits[1]) > 0, "phi_range must be positive"
        self.limits = limits

    @property
    def _pack_data(self):
        return super()._pack_data + [self.limits.view(4).contiguous()]

    def isect_gs_tiles(self, points, scale, rotation, width: int, height: int, flags, radii, means2d, depths,
                       points_velocity=None, opacity=None, tile_size_x: int = 16, tile_size_y: int = 16,
                       ut_alpha: float = 0.1, ut_beta: float = 2.0, ut_kappa: float = 0.0, sort: bool = True,
                       double_buffer: bool = True, tile_offsets=None, keys: bool = True):
        return isect_spherical_tiles(camera_pack=self.pack, points=points, points_velocity=points_velocity,
                                     scale=scale, quat=rotation, opacity=opacity, flag=flags, means2d=means2d,
                                     radii=radii, depths=depths, tile_size_x=tile_size_x, tile_size_y=tile_size_y,
                                     img_width=width, img_height=height, ut_alpha=ut_alpha, ut_beta=ut_beta,
                                     ut_kappa=ut_kappa, sort=sort, double_buffer=double_buffer,
                                     tile_offsets=tile_offsets, keys=keys)
