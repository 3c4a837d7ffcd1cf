"""LidarCamera: reference src/xsimgs/cameras/ext/lidar.py:14-83 and the beam / limit construction of
cameras/torch/lidar.py:8-57. The pack carries the device address of ``beam_v`` as two float32
bit patterns; the caller keeps ``beam_v`` alive while the pack is in use."""
import numpy as np
import torch

from .._C import LidarCamera as CLidarCamera, isect_lidar_tiles
from .ext_camera import CameraPose, FusedRSCamera


def data_addr_tensor(src_t: torch.Tensor) -> torch.Tensor:
    data_ptr = src_t.data_ptr()
    b1 = data_ptr & 0xffffffff
    b2 = data_ptr >> 32
    arr = np.array([b1, b2], dtype=np.uint32).view(np.float32)
    return torch.tensor(arr, device=src_t.device)


def cornering_values_from_pixel_values(vmin, vmax, img_size: int):
    rescale = 0.5 / (img_size - 0.5)
    b = (vmin - vmax * rescale) / (1 - rescale)
    a = 2 * (vmin - b)
    return b, a * img_size + b


def lidar_limits_from_beams(beam_angles: torch.Tensor, phi_min: float = 0.0, phi_range: float = 2 * np.pi):
    """limits and beam_v as LidarCameraTorch.create computes them (top beam first)."""
    num_beams = beam_angles.shape[-1]
    theta_min, theta_max = cornering_values_from_pixel_values(beam_angles.amax(dim=-1), beam_angles.amin(dim=-1),
                                                              num_beams)
    theta_min = theta_min.clamp(-torch.pi / 2, torch.pi / 2)
    theta_max = theta_max.clamp(-torch.pi / 2, torch.pi / 2)
    theta_range = theta_max - theta_min
    limits = torch.stack([torch.as_tensor(phi_min, dtype=theta_min.dtype),
                          torch.as_tensor(phi_range, dtype=theta_min.dtype), theta_min, theta_range], dim=-1)
    beam_v = (beam_angles.contiguous() - theta_min) / theta_range
    return limits, beam_v


class LidarCamera(FusedRSCamera):
    ext_cls = CLidarCamera

    def __init__(self, pose: CameraPose, limits: torch.Tensor, beam_v: torch.Tensor):
        super().__init__(pose)
        dev = pose.q.device
        self.limits = torch.as_tensor(limits, dtype=torch.float32, device=dev).reshape(4).contiguous()
        self.beam_v = torch.as_tensor(beam_v, dtype=torch.float32, device=dev).contiguous()

    @classmethod
    def create(cls, pose: CameraPose, beam_angles: torch.Tensor, phi_min: float = 0.0,
               phi_range: float = 2 * np.pi):
        limits, beam_v = lidar_limits_from_beams(beam_angles.float().cpu(), phi_min, phi_range)
        return cls(pose, limits, beam_v)

    @property
    def num_beams(self):
        return self.beam_v.shape[-1]

    def _beam_addr(self):
        """The pack's address tensor for ``beam_v``, rebuilt only when ``beam_v`` moves: building it is a
        host-to-device copy from pageable memory, which waits for every kernel already queued, so one
        per pack kept the host from queueing a frame ahead of the GPU. (It holds the address alone,
        which in-place changes of the beam values leave as it is.)"""
        ptr = self.beam_v.data_ptr()
        if self.__dict__.get("_addr_ptr") != ptr:
            self._addr = data_addr_tensor(self.beam_v)
            self._addr_ptr = ptr
        return self._addr

    @property
    def _pack_data(self):
        if not self.beam_v.is_contiguous():
            self.beam_v = self.beam_v.contiguous()
        return super()._pack_data + [self.limits.view(4).contiguous(), self._beam_addr()]

    def isect_gs_tiles(self, points, scale, rotation, width: int, height: int, flags, radii, means2d, depths,
                       points_velocity=None, opacity=None, tile_size_x: int = 16, tile_size_y: int = 16,
                       ut_alpha: float = 0.1, ut_beta: float = 2.0, ut_kappa: float = 0.0, sort: bool = True,
                       double_buffer: bool = True, tile_offsets=None, keys: bool = True):
        elev_boundaries = self.beam_v[::tile_size_y].contiguous()
        return isect_lidar_tiles(camera_pack=self.pack, points=points, points_velocity=points_velocity, scale=scale,
                                 quat=rotation, opacity=opacity, flag=flags, means2d=means2d, radii=radii,
                                 depths=depths, elev_boundaries=elev_boundaries, tile_size_x=tile_size_x,
                                 img_width=width, img_height=height, ut_alpha=ut_alpha, ut_beta=ut_beta,
                                 ut_kappa=ut_kappa, sort=sort, double_buffer=double_buffer,
                                 tile_offsets=tile_offsets, keys=keys)
