"""Camera front-end (reference src/xsimgs/cameras/ext, without the toast dependency)."""
from .ext_camera import CameraPose, FusedRSCamera
from .perspective import PerspectiveCamera
from .distorted_perspective import DistortedPerspectiveCamera, max_valid_radius
from .fisheye import FisheyeCamera
from .spherical import SphericalCamera
from .lidar import LidarCamera, data_addr_tensor, lidar_limits_from_beams

__all__ = ["CameraPose", "FusedRSCamera", "PerspectiveCamera", "DistortedPerspectiveCamera", "FisheyeCamera",
           "SphericalCamera", "LidarCamera", "data_addr_tensor", "lidar_limits_from_beams", "max_valid_radius"]
