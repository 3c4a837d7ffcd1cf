"""One training frame of the hot path, as the reference's caller runs it.

activations (exp scales, sigmoid opacity: one fused launch, its gradients another) -> camera rays ->
UT projection -> tile binning with sort -> per-tile offsets -> SH colours -> eval3d composite forward
-> composite backward -> SH backward -> activation gradients. The sequence is ut_gs_render's
(reference src/xsimgs/rendering/render.py:85-187) with the intermediates kept for inspection; the
activations and the SH call are the caller's, as in the reference, whose caller evaluates the colours
first: here they come after the projection, for the Gaussians some tile can hold only (the SH mask),
which gives the same images and gradients. render_rig keeps the colours first and unmasked: over a
rig most Gaussians are in some camera's view, and the mask there cost more than it saved.
"""
from __future__ import annotations

import contextlib
from dataclasses import dataclass, field

import torch

from . import cameras as C
from ._C import isect_regular_tiles_batched, packed_visibility_mask
from .rendering.activate import activate_gaussians
from .rendering.rasterize import ut_gs_rasterize, ut_gs_rasterize_batched
from .rendering.render import ut_gs_tiling
from .rendering.sh import spherical_harmonics_fused


@dataclass
class FrameState:
    scene: object
    device: torch.device
    means: torch.Tensor
    log_scales: torch.Tensor
    quats: torch.Tensor
    opacity_logits: torch.Tensor
    sh: torch.Tensor | None
    colors: torch.Tensor | None
    cams: list = field(default_factory=list)


def make_camera(spec, device) -> C.FusedRSCamera:
    pose = C.CameraPose.make(q=spec.q, t=spec.t, v=spec.v, w=spec.w, duration=spec.rolling,
                             offset_time=spec.trigger_time, pose_time=spec.pose_time, device=device)
    if spec.kind == "pinhole":
        return C.PerspectiveCamera(pose, torch.tensor(spec.impl))
    if spec.kind == "spherical":
        return C.SphericalCamera(pose, torch.tensor(spec.impl))
    if spec.kind == "distorted":
        cam = C.DistortedPerspectiveCamera(pose, torch.tensor(spec.impl), torch.tensor(spec.dist))
        if spec.max_radius is not None:
            cam._max_radius = torch.tensor([float(spec.max_radius)], device=device)
        return cam
    if spec.kind == "fisheye":
        return C.FisheyeCamera(pose, torch.tensor(spec.impl), torch.tensor(spec.dist))
    return C.LidarCamera(pose, torch.tensor(spec.impl), spec.beam_v)


def prepare(scene, device, requires_grad: bool = True) -> FrameState:
    def leaf(t):
        if t is None:
            return None
        return t.to(device).contiguous().requires_grad_(requires_grad)

    st = FrameState(scene, torch.device(device), leaf(scene.means), leaf(scene.log_scales), leaf(scene.quats),
                    leaf(scene.opacity_logits), leaf(scene.sh_coeffs), leaf(scene.colors))
    st.cams = [make_camera(spec, device) for spec in scene.cameras]
    return st


def render_frame(st: FrameState, backward: bool = False, grads=None, cam_index: int = 0) -> dict:
    sc = st.scene
    spec = sc.cameras[cam_index]
    cam = st.cams[cam_index]
    scales, opac = activate_gaussians(st.log_scales, st.opacity_logits)
    tsx, tsy = sc.tile_size
    with cam._freeze_ctx():
        ray_o, ray_d = cam.camera_rays(spec.width, spec.height, normalized_rays=True, return_origins=True,
                                       world_space=True)
        tiles = ut_gs_tiling(cam, st.means, scales, st.quats, spec.width, spec.height, opacity=opac,
                             tile_size_x=tsx, tile_size_y=tsy, use_phm=sc.use_phm)
        colors = _colors(st, cam.pose.t, tiles["radii"] if spec.kind in REGULAR_TILING else None)
        rgb, depth, alpha = ut_gs_rasterize(st.means, st.quats, scales, opac, colors, ray_o, ray_d,
                                            tiles["isect_offsets"], tiles["flatten_ids"], tsx, tsy)
    out = dict(rgb=rgb, depth=depth, alpha=alpha, colors=colors, ray_o=ray_o, ray_d=ray_d,
               offsets=tiles["isect_offsets"], flatten_ids=tiles["flatten_ids"], radii=tiles["radii"],
               means2d=tiles["means2d"], depths=tiles["depth"])
    if backward:
        g_rgb, g_depth, g_alpha = [g.to(st.device) for g in grads]
        torch.autograd.backward([rgb, depth, alpha], [g_rgb, g_depth, g_alpha])
        out["grads"] = dict(means=st.means.grad, quats=st.quats.grad, log_scales=st.log_scales.grad,
                            opacity_logits=st.opacity_logits.grad,
                            sh=st.sh.grad if st.sh is not None else None,
                            colors=st.colors.grad if st.colors is not None else None)
    return out


REGULAR_TILING = ("pinhole", "distorted", "fisheye")


def rig_batchable(st: FrameState) -> bool:
    """Cameras whose frame can run batched: regular tiling and one image size (the scenes here are
    static; camera motion only enters the per-camera projections and rays)."""
    specs = st.scene.cameras
    return (len(specs) > 1 and all(s.kind in REGULAR_TILING for s in specs)
            and len({(s.width, s.height) for s in specs}) == 1)


def rig_shares_origin(st: FrameState) -> bool:
    """Every camera at one origin: view-dependent colours are then the same for all of them."""
    return len({tuple(float(x) for x in s.t) for s in st.scene.cameras}) == 1


def render_rig(st: FrameState, backward: bool = False, grads=None) -> dict:
    """Every camera of a rig in one batched pass (an extension of this build; the reference's caller
    renders one camera per call, render.py:85-187). Per camera the UT projection and the rays, as
    in render_frame; then one batched binning (keys carry the camera above the tile bits), one
    compositor launch per pass over all cameras' tiles and, when the cameras share their origin,
    one SH evaluation whose colours every camera uses (its gradient sums over the cameras).
    grads: ([C, H, W, ch], [C, H, W], [C, H, W]) image gradients."""
    sc = st.scene
    specs = sc.cameras
    if not rig_batchable(st):
        raise ValueError("render_rig takes a static rig of regular-tiling cameras of one image size")
    W, H = specs[0].width, specs[0].height
    scales, opac = activate_gaussians(st.log_scales, st.opacity_logits)
    if st.sh is None:
        colors = st.colors
    elif rig_shares_origin(st):
        colors = spherical_harmonics_fused(st.sh, st.means, st.cams[0].pose.t, sc.sh_degree)
    else:
        colors = torch.stack([spherical_harmonics_fused(st.sh, st.means, cam.pose.t, sc.sh_degree)
                              for cam in st.cams])
    tsx, tsy = sc.tile_size
    ntx, nty = (W + tsx - 1) // tsx, (H + tsy - 1) // tsy
    C, N = len(specs), st.means.shape[0]
    dev = st.device
    # every camera's rays go straight into its slice of the rig's buffers; cameras of one kind project
    # in one launch that reads each Gaussian once, others one camera at a time into their slices
    ray_o = torch.empty((C, H, W, 3), device=dev)
    ray_d = torch.empty((C, H, W, 3), device=dev)
    one_kind = len({type(cam) for cam in st.cams}) == 1
    with torch.no_grad(), contextlib.ExitStack() as frozen:
        for cam in st.cams:
            frozen.enter_context(cam._freeze_ctx())
        for c, cam in enumerate(st.cams):
            cam.camera_rays(W, H, normalized_rays=True, return_origins=True, world_space=True,
                            out=(ray_o[c], ray_d[c]))
        if one_kind:
            cam0 = st.cams[0]
            flags, radii, means2d, depths = cam0.ext_cls.projection_utgs_rig(
                torch.cat([cam.pack for cam in st.cams]), st.means.contiguous(), None, scales.contiguous(),
                st.quats.contiguous(), opac.contiguous(), width=W, height=H,
                residual_thr_early_stop=cam0.residual_thr_early_stop, max_residual=cam0.residual_max_valid,
                max_margin=cam0.max_margin)
        else:
            flags = torch.empty((C, N), dtype=torch.uint8, device=dev)
            radii = torch.empty((C, N, 2), device=dev)
            means2d = torch.empty((C, N, 2), device=dev)
            depths = torch.empty((C, N), device=dev)
            for c, cam in enumerate(st.cams):
                cam.ut_gs_projection(st.means, scales, st.quats, W, H, opacity=opac, use_phm=sc.use_phm,
                                     out=(flags[c], radii[c], means2d[c], depths[c]))
        offsets = torch.empty((len(specs), nty, ntx), dtype=torch.int32, device=st.device)
        _, _, flatten_ids = isect_regular_tiles_batched(means2d, radii, depths, W, H, tsx, tsy, sort=True,
                                                        tile_offsets=offsets, keys=False)
    rgb, depth, alpha = ut_gs_rasterize_batched(st.means, st.quats, scales, opac, colors, ray_o, ray_d, offsets,
                                                flatten_ids, tsx, tsy)
    out = dict(rgb=rgb, depth=depth, alpha=alpha, colors=colors, ray_o=ray_o, ray_d=ray_d, offsets=offsets,
               flatten_ids=flatten_ids, radii=radii, means2d=means2d, depths=depths)
    if backward:
        g_rgb, g_depth, g_alpha = [g.to(st.device) for g in grads]
        torch.autograd.backward([rgb, depth, alpha], [g_rgb, g_depth, g_alpha])
        out["grads"] = dict(means=st.means.grad, quats=st.quats.grad, log_scales=st.log_scales.grad,
                            opacity_logits=st.opacity_logits.grad,
                            sh=st.sh.grad if st.sh is not None else None,
                            colors=st.colors.grad if st.colors is not None else None)
    return out


def _colors(st: FrameState, origin, radii=None):
    """The Gaussians' colours: SH evaluated at the origin, or the fixed colours. With the radii of a
    regular tiling's projection ([N, 2], or [C, N, 2] for all the cameras of one origin), only the
    Gaussians some tile can hold are evaluated (the SH mask; the others' colours are zeros). The
    compositor reads no other Gaussian's colour, so the images are the same and so are the gradients
    (the others' colour gradients are zeros either way)."""
    if st.sh is None:
        return st.colors
    mask = packed_visibility_mask(radii.detach().contiguous()) if radii is not None else None
    return spherical_harmonics_fused(st.sh, st.means, origin, st.scene.sh_degree, mask=mask)


def zero_grads(st: FrameState) -> None:
    for t in (st.means, st.log_scales, st.quats, st.opacity_logits, st.sh, st.colors):
        if t is not None:
            t.grad = None
