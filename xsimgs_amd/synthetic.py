"""Seeded synthetic scenes for the benchmark configurations.

Every tensor is drawn on the CPU from one ``torch.Generator`` in a fixed order
(means, log-scales, quaternions, opacity logits, SH DC, SH rest, extra
per-config tensors, upstream gradients) in float32, so that the GPU path and
the CPU oracle see bit-identical inputs after a copy to the device.

Configurations (0-based, as listed by the benchmark definition):

* ``cfg0`` -- 10k Gaussians, SH0, one 256x256 pinhole camera, forward only.
* ``cfg1`` -- 1M Gaussians, SH3, 1920x1080 pinhole camera, forward only.
* ``cfg2`` -- the ``cfg1`` scene, forward+backward (the headline frame).
* ``cfg3`` -- 3M Gaussians on a ring, 2048x128 spherical lidar, CDIM=2.
* ``cfg4`` -- 4M Gaussians in 2000 blobs, six 1600x900 pinhole cameras.

Camera conventions follow the reference camera model: a camera point
``(x, y, z)`` projects to ``u = x fx / z + cx`` (x right, y down, z forward);
poses are camera-to-world quaternions stored ``(w, x, y, z)``
(reference ``include/cameras/projection_kernels.h:74-113``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch


@dataclass
class CameraSpec:
    """Plain description of one camera, independent of any device."""

    kind: str                      # "pinhole" | "spherical" | "lidar" | "distorted" | "fisheye"
    width: int
    height: int
    q: list                        # camera-to-world rotation (w, x, y, z)
    t: list                        # camera position in world
    impl: list                     # pinhole, distorted, fisheye: [fx/W, fy/H, cx/W, cy/H]; spherical: limits
    v: list = field(default_factory=lambda: [0.0, 0.0, 0.0])
    w: list = field(default_factory=lambda: [0.0, 0.0, 0.0])
    rolling: list = field(default_factory=lambda: [0.0, 0.0])
    trigger_time: float = 0.0
    pose_time: float = 0.0
    beam_v: torch.Tensor | None = None   # lidar only: per-row v values
    dist: list | None = None       # distorted: k1 k2 p1 p2 k3 k4 k5 k6; fisheye: k1 k2 k3 k4
    max_radius: float | None = None  # distorted: largest camera-space radius |xy / z| projected


@dataclass
class Scene:
    name: str
    means: torch.Tensor            # [N, 3]
    log_scales: torch.Tensor       # [N, 3]
    quats: torch.Tensor            # [N, 4] (w, x, y, z), unit
    opacity_logits: torch.Tensor   # [N]
    sh_coeffs: torch.Tensor | None # [N, K, 3]
    sh_degree: int
    colors: torch.Tensor | None    # [N, CDIM] explicit features (lidar)
    cameras: list
    tile_size: tuple
    backward: bool
    grad_rgb: list = field(default_factory=list)    # per camera [H, W, C]
    grad_depth: list = field(default_factory=list)  # per camera [H, W]
    grad_alpha: list = field(default_factory=list)  # per camera [H, W]
    use_phm: bool = False
    notes: str = ""

    @property
    def n(self) -> int:
        return self.means.shape[0]

    @property
    def scales(self) -> torch.Tensor:
        return torch.exp(self.log_scales)

    @property
    def opacity(self) -> torch.Tensor:
        return torch.sigmoid(self.opacity_logits)


def _quat_mul(a, b):
    aw, ax, ay, az = a
    bw, bx, by, bz = b
    return [aw * bw - ax * bx - ay * by - az * bz,
            aw * bx + ax * bw + ay * bz - az * by,
            aw * by - ax * bz + ay * bw + az * bx,
            aw * bz + ax * by - ay * bx + az * bw]


def _axis_angle_quat(axis, angle):
    s = math.sin(0.5 * angle)
    return [math.cos(0.5 * angle), axis[0] * s, axis[1] * s, axis[2] * s]


def pinhole(width, height, fx, fy, cx, cy, q=(1.0, 0.0, 0.0, 0.0), t=(0.0, 0.0, 0.0)):
    return CameraSpec("pinhole", width, height, list(q), list(t),
                      [fx / width, fy / height, cx / width, cy / height])


def _unit_quats(g, n):
    q = torch.randn(n, 4, generator=g)
    return q / q.norm(dim=-1, keepdim=True)


def _grads(g, cams, cdim):
    rgb, dep, alp = [], [], []
    for c in cams:
        rgb.append(torch.randn(c.height, c.width, cdim, generator=g) * 1e-3)
        alp.append(torch.randn(c.height, c.width, generator=g) * 1e-3)
        dep.append(torch.randn(c.height, c.width, generator=g) * 1e-3)
    return rgb, dep, alp


def make_cfg0(seed: int = 0, n: int = 10_000, width: int = 256, height: int = 256) -> Scene:
    g = torch.Generator("cpu").manual_seed(seed)
    lo = torch.tensor([-5.0, -2.0, 2.0])
    hi = torch.tensor([5.0, 2.0, 20.0])
    means = lo + (hi - lo) * torch.rand(n, 3, generator=g)
    log_s = -3.0 + 0.5 * torch.randn(n, 3, generator=g)
    quats = _unit_quats(g, n)
    op = 1.5 * torch.randn(n, generator=g)
    dc = 0.3 * torch.randn(n, 1, 3, generator=g)
    cam = pinhole(width, height, 256.0 * width / 256, 256.0 * height / 256,
                  width / 2, height / 2)
    return Scene("cfg0", means, log_s, quats, op, dc, 0, None, [cam], (16, 16), False,
                 notes="near/far (0.01, 100) have no counterpart in the projection")


def _sh3(g, n):
    dc = 0.3 * torch.randn(n, 1, 3, generator=g)
    rest = 0.05 * torch.randn(n, 15, 3, generator=g)
    return torch.cat([dc, rest], dim=1)


def make_cfg1(seed: int = 0, n: int = 1_000_000, backward: bool = False, frustum: bool = False) -> Scene:
    """``frustum``: lateral positions confined to the camera's field of view (x, y ~ U(-1, 1) times
    the half-extent of the image at that depth) instead of U(-1.2, 1.2) * depth, so that every
    Gaussian is in view."""
    g = torch.Generator("cpu").manual_seed(seed)
    u = torch.rand(n, 3, generator=g)
    z = torch.exp(math.log(2.0) + (math.log(80.0) - math.log(2.0)) * u[:, 2])
    sx, sy = (960.0 / 1728.0, 540.0 / 1728.0) if frustum else (1.2, 1.2)
    x = (2.0 * u[:, 0] - 1.0) * sx * z
    y = (2.0 * u[:, 1] - 1.0) * sy * z
    means = torch.stack([x, y, z], dim=-1)
    log_s = -3.0 + 0.7 * torch.randn(n, 3, generator=g)
    quats = _unit_quats(g, n)
    op = 1.5 * torch.randn(n, generator=g)
    sh = _sh3(g, n)
    cam = pinhole(1920, 1080, 1728.0, 1728.0, 960.0, 540.0)
    sc = Scene(("cfg2" if backward else "cfg1") + ("_frustum" if frustum else ""), means, log_s, quats, op, sh, 3,
               None, [cam], (16, 16), backward,
               notes=("lateral spread confined to the field of view" if frustum else
                      "lateral spread read literally: x, y ~ U(-1.2, 1.2) * depth"))
    if backward:
        sc.grad_rgb, sc.grad_depth, sc.grad_alpha = _grads(g, [cam], 3)
    return sc


def make_cfg2(seed: int = 0, n: int = 1_000_000, frustum: bool = False) -> Scene:
    return make_cfg1(seed, n, backward=True, frustum=frustum)


def make_cfg2_frustum(seed: int = 0, n: int = 1_000_000) -> Scene:
    return make_cfg1(seed, n, backward=True, frustum=True)


def lidar_beams(n_beams: int = 128, top_deg: float = 15.0, bottom_deg: float = -25.0):
    """Beam elevations (radians) from the top beam down, and the derived limits.

    Follows ``LidarCameraTorch.create`` (reference
    ``src/xsimgs/cameras/torch/lidar.py:27-57``): the elevation range is extended
    by half a beam on both sides so the limits describe image corners, and
    ``beam_v`` is the normalised v coordinate of each beam (increasing, because
    ``theta_range`` is negative for a top-first beam order).
    """
    ang = torch.linspace(math.radians(top_deg), math.radians(bottom_deg), n_beams)
    vmin = ang.max()
    vmax = ang.min()
    rescale = 0.5 / (n_beams - 0.5)
    b = (vmin - vmax * rescale) / (1 - rescale)
    a = 2 * (vmin - b)
    theta_min = torch.clamp(b, -math.pi / 2, math.pi / 2)
    theta_max = torch.clamp(a * n_beams + b, -math.pi / 2, math.pi / 2)
    theta_range = theta_max - theta_min
    beam_v = (ang - theta_min) / theta_range
    limits = [0.0, 2.0 * math.pi, float(theta_min), float(theta_range)]
    return ang, beam_v.contiguous(), limits


def make_cfg3(seed: int = 0, n: int = 3_000_000, width: int = 2048, n_beams: int = 128) -> Scene:
    g = torch.Generator("cpu").manual_seed(seed)
    u = torch.rand(n, 3, generator=g)
    r = torch.exp(math.log(1.0) + (math.log(120.0) - math.log(1.0)) * u[:, 0])
    az = 2.0 * math.pi * u[:, 1]
    z = -2.0 + 8.0 * u[:, 2]
    means = torch.stack([r * torch.cos(az), r * torch.sin(az), z], dim=-1)
    log_s = -2.5 + 0.7 * torch.randn(n, 3, generator=g)
    quats = _unit_quats(g, n)
    op = 1.5 * torch.randn(n, generator=g)
    intensity = torch.rand(n, generator=g)
    drop_logit = torch.randn(n, generator=g)
    colors = torch.stack([intensity, drop_logit], dim=-1)
    _, beam_v, limits = lidar_beams(n_beams)
    cam = CameraSpec("lidar", width, n_beams, [1.0, 0.0, 0.0, 0.0], [0.0, 0.0, 0.0], limits,
                     beam_v=beam_v)
    sc = Scene("cfg3", means, log_s, quats, op, None, 0, colors, [cam], (32, 8), True,
               use_phm=True,
               notes="colors = [intensity ~ U(0,1), ray-drop logit ~ N(0,1)]")
    sc.grad_rgb, sc.grad_depth, sc.grad_alpha = _grads(g, [cam], 2)
    return sc


def rig_cameras(width=1600, height=900, f=1260.0, n_cams=6):
    """Six pinhole cameras at the origin, yawed 0/60/.../300 deg about world +z.

    World frame is z-up; the yaw-0 camera looks along world +x with its image x
    axis along world -y and image y axis along world -z.
    """
    base = [0.5, -0.5, 0.5, -0.5]  # maps cam z->world x, cam x->world -y, cam y->world -z
    cams = []
    for i in range(n_cams):
        yaw = math.radians(60.0 * i)
        q = _quat_mul(_axis_angle_quat([0.0, 0.0, 1.0], yaw), base)
        cams.append(pinhole(width, height, f, f, width / 2, height / 2, q=q))
    return cams


def make_cfg4(seed: int = 0, n: int = 4_000_000, n_blobs: int = 2000) -> Scene:
    g = torch.Generator("cpu").manual_seed(seed)
    # blob centres: ring, horizontal range U(5, 60) m, azimuth U(0, 2pi), z U(-2, 6)
    cu = torch.rand(n_blobs, 3, generator=g)
    cr = 5.0 + 55.0 * cu[:, 0]
    caz = 2.0 * math.pi * cu[:, 1]
    cz = -2.0 + 8.0 * cu[:, 2]
    centres = torch.stack([cr * torch.cos(caz), cr * torch.sin(caz), cz], dim=-1)
    blob = torch.randint(0, n_blobs, (n,), generator=g)
    means = centres[blob] + 1.5 * torch.randn(n, 3, generator=g)
    log_s = -3.0 + 0.7 * torch.randn(n, 3, generator=g)
    quats = _unit_quats(g, n)
    op = 1.0 + torch.randn(n, generator=g)
    sh = _sh3(g, n)
    cams = rig_cameras()
    sc = Scene("cfg4", means, log_s, quats, op, sh, 3, None, cams, (16, 16), True,
               notes="blob centres on a ring, range U(5,60) m, z U(-2,6); log-scales N(-3,0.7)")
    sc.grad_rgb, sc.grad_depth, sc.grad_alpha = _grads(g, cams, 3)
    return sc


MAKERS = {"cfg0": make_cfg0, "cfg1": make_cfg1, "cfg2": make_cfg2,
          "cfg3": make_cfg3, "cfg4": make_cfg4, "cfg2_frustum": make_cfg2_frustum}


def make(name: str, **kw) -> Scene:
    return MAKERS[name](**kw)
