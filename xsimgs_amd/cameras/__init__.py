"""Camera front-end (reference src/xsimgs/cameras/ext, without the toast dependency)."""
from .ext_camera import CameraPose, FusedRSCamera
from .perspective import PerspectiveCamera
from .spherical import SphericalCamera
from .lidar import LidarCamera, data_addr_tensor, lidar_limits_from_beams

__all__ = ["CameraPose", "FusedRSCamera", "PerspectiveCamera", "SphericalCamera", "LidarCamera",
           "data_addr_tensor", "lidar_limits_from_beams"]
