"""FusedRSCamera: reference src/xsimgs/cameras/ext/ext_camera.py:8-210.

The reference builds camera state from toast objects (LinearMotion, RollingShutter); this
front-end holds the same seven tensors directly (``CameraPose``) and produces the same pack
order: q(4), t(3), v(3), w(3), shutter duration(2), shutter offset time(1), pose time(1),
followed by the camera model's own tensors (ext_camera.py:17-26).
"""
from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass

import torch

from .._C import isect_regular_tiles


def _t(x, n, device, dtype=torch.float32):
    t = torch.as_tensor(x, dtype=dtype, device=device).reshape(n)
    return t.contiguous()


@dataclass
class CameraPose:
    """Camera-to-world pose (quaternion w, x, y, z), its linear / angular velocity and the
    rolling-shutter timing (duration along u and v, trigger offset time, pose time)."""

    q: torch.Tensor
    t: torch.Tensor
    v: torch.Tensor
    w: torch.Tensor
    duration: torch.Tensor
    offset_time: torch.Tensor
    pose_time: torch.Tensor

    @classmethod
    def make(cls, q=(1.0, 0.0, 0.0, 0.0), t=(0.0, 0.0, 0.0), v=(0.0, 0.0, 0.0), w=(0.0, 0.0, 0.0),
             duration=(0.0, 0.0), offset_time=0.0, pose_time=0.0, device="cuda"):
        return cls(_t(q, 4, device), _t(t, 3, device), _t(v, 3, device), _t(w, 3, device),
                   _t(duration, 2, device), _t([offset_time], 1, device), _t([pose_time], 1, device))


class FusedRSCamera:
    ext_cls = None
    use_phm: bool = False

    residual_thr_early_stop: float = 1e-4
    residual_max_valid: float = 0.002
    max_margin: float = 1.0

    def __init__(self, pose: CameraPose):
        self.pose = pose
        self._pack = None
        self._freeze_flag = False

    @property
    def device(self):
        return self.pose.q.device

    @property
    def _pack_data(self) -> list:
        p = self.pose
        return [p.q.view(4).contiguous(), p.t.view(3).contiguous(), p.v.view(3).contiguous(),
                p.w.view(3).contiguous(), p.duration.view(2).contiguous(), p.offset_time.view(1),
                p.pose_time.view(1)]

    def _set_freeze(self, value: bool):
        self._freeze_flag = value
        self._pack = None

    @contextmanager
    def _freeze_ctx(self):
        needed = not self._freeze_flag
        if needed:
            self._set_freeze(True)
        try:
            yield
        finally:
            if needed:
                self._set_freeze(False)

    @classmethod
    def supports_phm(cls) -> bool:
        return hasattr(cls.ext_cls, "projection_utgs_phm")

    @property
    def pack(self):
        if self._freeze_flag and self._pack is not None:
            return self._pack
        self._pack = self.ext_cls.pack(self._pack_data)
        return self._pack

    def world_to_uv(self, points, points_velocity=None, points_time=None):
        if points_time is not None and points_velocity is not None:
            delta_t = points_time - self.pose.pose_time
            points = points + delta_t * points_velocity
        return self.ext_cls.projection(
            self.pack, points.contiguous(),
            points_velocity.contiguous() if points_velocity is not None else None,
            residual_thr_early_stop=self.residual_thr_early_stop, max_residual=self.residual_max_valid,
            max_margin=self.max_margin)

    def camera_rays(self, width: int, height: int, normalized_rays: bool = True, world_space: bool = True,
                    return_origins: bool = True, return_valid: bool = False, out=None):
        """out (extension): preallocated (ray_o, ray_d) tensors of [height, width, 3] to write into."""
        out = self.ext_cls.camera_rays(self.pack, width=width, height=height, world_space=world_space,
                                       normalized=normalized_rays, return_origins=return_origins,
                                       return_valid=return_valid, out=out)
        ray_o = out[0] if return_origins else None
        if return_valid:
            return ray_o, out[1], out[2]
        return ray_o, out[1]

    def uv_time(self, uv):
        return self.ext_cls.pixel_time_from_uv(self.pack, uv.contiguous()).unsqueeze(-1)

    def uv_time_delta(self, uv):
        return self.ext_cls.pixel_time_delta_from_uv(self.pack, uv.contiguous()).unsqueeze(-1)

    def image_time(self, image):
        return self.ext_cls.pixel_time(self.pack, width=image.shape[1], height=image.shape[0]).unsqueeze(-1)

    def image_time_delta(self, image):
        return self.ext_cls.pixel_time_delta(self.pack, width=image.shape[1], height=image.shape[0]).unsqueeze(-1)

    def undistort_map(self, width: int, height: int, normalized_range: bool = False):
        if not hasattr(self.ext_cls, "undistort_map"):
            raise NotImplementedError(f'Camera extension class "{self.ext_cls.__name__}" does not implement '
                                      '"undistort_map"')
        return self.ext_cls.undistort_map(self.pack, width=width, height=height, normalized_range=normalized_range)

    def ut_gs_projection(self, points, scale, rotation, width: int, height: int, points_velocity=None,
                         opacity=None, ut_alpha: float = 0.1, ut_beta: float = 2.0, ut_kappa: float = 0.0,
                         use_phm: bool = None, out=None):
        """out (extension): preallocated (flags, radii, means2d, depths) tensors to write into."""
        if use_phm is None:
            use_phm = self.use_phm
        proj_fn = (self.ext_cls.projection_utgs_phm if use_phm and self.supports_phm()
                   else self.ext_cls.projection_utgs)
        return proj_fn(self.pack, points.contiguous(),
                       points_velocity.contiguous() if points_velocity is not None else None,
                       scale.contiguous(), rotation.contiguous(),
                       opacity.contiguous() if opacity is not None else None, width=width, height=height,
                       ut_alpha=ut_alpha, ut_beta=ut_beta, ut_kappa=ut_kappa,
                       residual_thr_early_stop=self.residual_thr_early_stop, max_residual=self.residual_max_valid,
                       max_margin=self.max_margin, out=out)

    def isect_gs_tiles(self, points, scale, rotation, width: int, height: int, flags, radii, means2d, depths,
                       points_velocity=None, opacity=None, tile_size_x: int = 16, tile_size_y: int = 16,
                       ut_alpha: float = 0.1, ut_beta: float = 2.0, ut_kappa: float = 0.0, sort: bool = True,
                       double_buffer: bool = True, tile_offsets=None, keys: bool = True):
        return isect_regular_tiles(means2d, radii, depths, img_width=width, img_height=height,
                                   tile_size_x=tile_size_x, tile_size_y=tile_size_y, sort=sort,
                                   double_buffer=double_buffer, tile_offsets=tile_offsets, keys=keys)
