"""Camera-pose gradients: the backward of camera rays and pixel times w.r.t. the camera.

CPU: the oracle's backward (oracle/xsg_oracle.c orc_camera_rays_bwd, orc_pixel_time_bwd) against
float64 central differences of its own forward, for every camera parameter. GPU: the HIP backward
(xsg_camera_rays_bwd, xsg_pixel_time_bwd) against the oracle, and the autograd path from the camera
tensors through the pack (`torch.cat`, whose backward is the reference's unpack_to_tensors).
"""
import copy

import numpy as np
import pytest
import torch

from oracle import oracle as O
from xsimgs_amd.synthetic import CameraSpec

W, H = 24, 14
FIELDS = O.CAMERA_GRAD_FIELDS


def _beam_v(n):
    return np.linspace(0.04, 0.97, n).astype(np.float32)


def _spec(kind, w_scale=1.0):
    q = np.array([0.92, 0.15, -0.25, 0.2])
    q = (q / np.linalg.norm(q)).tolist()
    common = dict(q=q, t=[1.0, -2.0, 0.5], v=[0.8, -0.3, 0.2], w=[0.9 * w_scale, -0.4 * w_scale, 0.6 * w_scale],
                  rolling=[0.03, 0.012], trigger_time=0.11, pose_time=0.13)
    if kind == "pinhole":
        return CameraSpec("pinhole", W, H, impl=[0.93, 1.41, 0.47, 0.53], **common)
    if kind == "spherical":
        return CameraSpec("spherical", W, H, impl=[0.1, 2.0 * np.pi, -0.6, 1.1], **common)
    if kind == "distorted":
        return CameraSpec("distorted", W, H, impl=[0.93, 1.41, 0.47, 0.53],
                          dist=[-0.28, 0.07, 1e-3, -5e-4, 0.01, 0.02, -0.004, 0.001], max_radius=1.5, **common)
    if kind == "fisheye":
        return CameraSpec("fisheye", W, H, impl=[0.35, 0.45, 0.5, 0.48], dist=[0.03, -0.005, 0.001, -0.0001],
                          **common)
    return CameraSpec("lidar", W, H, impl=[0.0, 2.0 * np.pi, 0.3, -0.7], beam_v=_beam_v(H), **common)


def _get(spec, name):
    if name == "max_radius_sq":
        return [float(spec.max_radius) ** 2]
    v = getattr(spec, name)
    return [float(v)] if np.isscalar(v) else [float(x) for x in v]


def _set(spec, name, vals):
    if name == "max_radius_sq":
        spec.max_radius = float(np.sqrt(vals[0]))
    else:
        setattr(spec, name, vals[0] if name in ("trigger_time", "pose_time") else list(vals))


def _loss(spec, go, gd, world_space, normalized):
    ro, rd = O.camera_rays(spec, W, H, world_space, normalized, prec="f64")
    return float((ro * go).sum() + (rd * gd).sum())


CASES = [(k, ws, nz, wsc) for k in ("pinhole", "spherical", "lidar") for ws in (True, False) for nz in (True, False)
         for wsc in (1.0, 1e-4)] + [(k, ws, nz, 1.0) for k in ("distorted", "fisheye") for ws in (True, False)
                                    for nz in (True, False)]


@pytest.mark.parametrize("kind,world_space,normalized,w_scale", CASES)
def test_oracle_ray_bwd_matches_finite_differences(kind, world_space, normalized, w_scale):
    spec = _spec(kind, w_scale)
    g = np.random.default_rng(3)
    go = g.standard_normal((H, W, 3))
    gd = g.standard_normal((H, W, 3))
    got = O.camera_rays_bwd(spec, W, H, go, gd, world_space, normalized, prec="f64")
    fd = []
    eps = 1e-6
    for name, n in O.camera_grad_fields(kind):
        base = _get(spec, name)
        for i in range(n):
            vals = list(base)
            sp, sm = copy.copy(spec), copy.copy(spec)
            vals[i] = base[i] + eps
            _set(sp, name, vals)
            vals[i] = base[i] - eps
            _set(sm, name, vals)
            fd.append((_loss(sp, go, gd, world_space, normalized) - _loss(sm, go, gd, world_space, normalized))
                      / (2 * eps))
    fd = np.array(fd)
    if kind in ("spherical", "lidar"):
        fd[17:] = 0.0  # the spherical and lidar models carry no intrinsics gradient (base_camera_impl.h:19-22)
    np.testing.assert_allclose(got, fd, rtol=1e-6, atol=1e-6 * max(1.0, np.abs(fd).max()))
    if not world_space:
        assert np.all(got[:17] == 0)


@pytest.mark.parametrize("kind", ["pinhole", "lidar"])
@pytest.mark.parametrize("delta", [False, True])
def test_oracle_pixel_time_bwd_closed_form(kind, delta):
    spec = _spec(kind)
    g = np.random.default_rng(4)
    grad = g.standard_normal((H, W))
    out = O.pixel_time_bwd(spec, grad, W, H, delta=delta, prec="f64")
    uv = O.pixel_uv(spec, W, H)
    want = np.zeros(21)
    want[13], want[14], want[15] = (grad * uv[..., 0]).sum(), (grad * uv[..., 1]).sum(), grad.sum()
    if delta:
        want[16] = -grad.sum()
    np.testing.assert_allclose(out, want, rtol=1e-12, atol=1e-12)
    # from uv: linear in uv with slope `rolling`
    uvs = g.uniform(0, 1, (37, 2))
    gg = g.standard_normal(37)
    out2, d_uv = O.pixel_time_bwd(spec, gg, uv=uvs, delta=delta, prec="f64")
    np.testing.assert_allclose(d_uv, gg[:, None] * np.array(spec.rolling)[None, :], rtol=1e-12)
    np.testing.assert_allclose(out2[15], gg.sum(), rtol=1e-12)


# ------------------------------------------------------------------ GPU: HIP backward vs oracle
def _gpu_cam(spec, dev, requires_grad=False):
    from xsimgs_amd import frame
    cam = frame.make_camera(spec, dev)
    if requires_grad:
        p = cam.pose
        for t in (p.q, p.t, p.v, p.w, p.duration, p.offset_time, p.pose_time):
            t.requires_grad_(True)
        if spec.kind != "lidar":
            _impl(cam).requires_grad_(True)
        if spec.kind in ("distorted", "fisheye"):
            cam.distortion.requires_grad_(True)
    return cam


def _impl(cam):
    return cam.normalized_intrinsics if hasattr(cam, "normalized_intrinsics") else cam.limits


def _close(got, ref, name):
    from tests._util import GRAD_ATOL, GRAD_RTOL, report
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    print(report(name, got, ref), flush=True)
    # the sum over pixels carries float32 rounding of order sqrt(pixels) * ulp of the largest term
    atol = GRAD_ATOL * max(1.0, np.abs(ref).max())
    bad = np.abs(got - ref) > atol + GRAD_RTOL * np.abs(ref)
    assert not bad.any(), (name, np.nonzero(bad)[0], got[bad], ref[bad])


GPU_RAY_CASES = [(k, ws, nz, ro) for k in ("pinhole", "spherical", "lidar", "distorted", "fisheye")
                 for ws in (True, False) for nz in (True, False) for ro in (True, False) if ws or ro]


@pytest.mark.gpu
@pytest.mark.parametrize("kind,world_space,normalized,return_origins", GPU_RAY_CASES)
def test_gpu_camera_rays_bwd(dev, kind, world_space, normalized, return_origins):
    print("case", kind, world_space, normalized, return_origins, flush=True)
    spec = _spec(kind)
    cam = _gpu_cam(spec, dev)
    pack = cam.pack.detach().clone().requires_grad_(True)
    out = cam.ext_cls.camera_rays(pack, W, H, world_space=world_space, normalized=normalized,
                                  return_origins=return_origins)
    g = np.random.default_rng(5)
    go = g.standard_normal((H, W, 3)).astype(np.float32)
    gd = g.standard_normal((H, W, 3)).astype(np.float32)
    loss = (out[1] * torch.from_numpy(gd).to(dev)).sum()
    if return_origins:
        loss = loss + (out[0] * torch.from_numpy(go).to(dev)).sum()
    loss.backward()
    got = pack.grad.detach().cpu().numpy().reshape(-1)
    assert got.shape[0] == {"lidar": 23, "distorted": 30, "fisheye": 25}.get(kind, 21)
    ref = O.camera_rays_bwd(spec, W, H, go if return_origins else None, gd, world_space, normalized, prec="f64")
    _close(got[:len(ref)], ref, f"d_pack {kind}")
    # the lidar beam-table address and the distorted model's max_radius^2 carry no gradient
    assert np.all(got[len(ref):] == 0)


@pytest.mark.gpu
@pytest.mark.parametrize("kind,size", [("pinhole", (1920, 1080)), ("lidar", (2048, 128))])
def test_gpu_camera_rays_bwd_full_frame(dev, kind, size):
    """A full frame: the deterministic two-level sum against the float64 oracle, and run-to-run
    bit equality."""
    w, h = size
    print("case", kind, size, flush=True)
    spec = _spec(kind)
    spec.width, spec.height = w, h
    if kind == "lidar":
        spec.beam_v = _beam_v(h)
    cam = _gpu_cam(spec, dev)
    g = torch.Generator().manual_seed(11)
    go = torch.randn(h, w, 3, generator=g)
    gd = torch.randn(h, w, 3, generator=g)
    grads = []
    for _ in range(2):
        pack = cam.pack.detach().clone().requires_grad_(True)
        ro, rd = cam.ext_cls.camera_rays(pack, w, h)
        ((ro * go.to(dev)).sum() + (rd * gd.to(dev)).sum()).backward()
        grads.append(pack.grad.detach().cpu().numpy().reshape(-1))
    assert np.array_equal(grads[0], grads[1])
    ref = O.camera_rays_bwd(spec, w, h, go.numpy(), gd.numpy(), True, True, prec="f64")
    _close(grads[0][:21], ref, f"d_pack full {kind}")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["pinhole", "spherical", "lidar", "distorted", "fisheye"])
def test_gpu_camera_grads_reach_pose_tensors(dev, kind):
    """Autograd from the rays to the camera's own tensors: the pack's backward splits the pack
    gradient over q, t, v, w, rolling, trigger, pose time and the intrinsics (pack_kernels.h:85-104)."""
    spec = _spec(kind)
    cam = _gpu_cam(spec, dev, requires_grad=True)
    ro, rd = cam.camera_rays(W, H)
    g = np.random.default_rng(6)
    go = g.standard_normal((H, W, 3)).astype(np.float32)
    gd = g.standard_normal((H, W, 3)).astype(np.float32)
    loss = (ro * torch.from_numpy(go).to(dev)).sum() + (rd * torch.from_numpy(gd).to(dev)).sum()
    loss.backward()
    ref = O.camera_rays_bwd(spec, W, H, go, gd, True, True, prec="f64")
    p = cam.pose
    got = np.concatenate([np.asarray(x.grad.detach().cpu().numpy()).reshape(-1)
                          for x in (p.q, p.t, p.v, p.w, p.duration, p.offset_time, p.pose_time)])
    if kind != "lidar":
        got = np.concatenate([got, _impl(cam).grad.detach().cpu().numpy().reshape(-1)])
    else:
        ref = ref[:17]
    if kind in ("distorted", "fisheye"):
        got = np.concatenate([got, cam.distortion.grad.detach().cpu().numpy().reshape(-1)])
        ref = ref[:len(got)]   # max_radius is derived from the coefficients, not a leaf
    _close(got, ref, f"pose grads {kind}")


@pytest.mark.gpu
@pytest.mark.parametrize("size", [(65, 33), (1, 300), (700, 1), (64, 32), (129, 97)])
def test_gpu_camera_grads_ragged_images(dev, size):
    """Image sizes around the 64 x 32 pixels each workgroup sums: partial strips and row blocks,
    single rows and columns, for the ray gradients and the per-pixel time gradients."""
    w, h = size
    print("case", size, flush=True)
    spec = _spec("distorted")
    spec.width, spec.height = w, h
    cam = _gpu_cam(spec, dev)
    g = np.random.default_rng(w * 1000 + h)
    go = g.standard_normal((h, w, 3)).astype(np.float32)
    gd = g.standard_normal((h, w, 3)).astype(np.float32)
    pack = cam.pack.detach().clone().requires_grad_(True)
    ro, rd = cam.ext_cls.camera_rays(pack, w, h)
    ((ro * torch.from_numpy(go).to(dev)).sum() + (rd * torch.from_numpy(gd).to(dev)).sum()).backward()
    ref = O.camera_rays_bwd(spec, w, h, go, gd, True, True, prec="f64")
    got = pack.grad.detach().cpu().numpy().reshape(-1)
    _close(got[:len(ref)], ref, f"d_pack {size}")
    for delta in (False, True):
        pack = cam.pack.detach().clone().requires_grad_(True)
        fn = cam.ext_cls.pixel_time_delta if delta else cam.ext_cls.pixel_time
        gr = g.standard_normal((h, w)).astype(np.float32)
        (fn(pack, w, h) * torch.from_numpy(gr).to(dev)).sum().backward()
        ref = O.pixel_time_bwd(spec, gr, w, h, delta=delta, prec="f64")
        _close(pack.grad.detach().cpu().numpy().reshape(-1)[:len(ref)], ref, f"d_pack time {size}")
    # many uvs: several 2048-element workgroups and a partial one
    pack = cam.pack.detach().clone().requires_grad_(True)
    uv_np = g.uniform(0, 1, (5000, 2)).astype(np.float32)
    uv = torch.from_numpy(uv_np).to(dev).requires_grad_(True)
    gr = g.standard_normal(5000).astype(np.float32)
    (cam.ext_cls.pixel_time_from_uv(pack, uv) * torch.from_numpy(gr).to(dev)).sum().backward()
    ref, ref_duv = O.pixel_time_bwd(spec, gr, uv=uv_np, prec="f64")
    _close(pack.grad.detach().cpu().numpy().reshape(-1)[:len(ref)], ref, "d_pack uv")
    _close(uv.grad.detach().cpu().numpy().reshape(-1), ref_duv.reshape(-1), "d_uv")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["pinhole", "lidar"])
@pytest.mark.parametrize("delta", [False, True])
@pytest.mark.parametrize("from_uv", [False, True])
def test_gpu_pixel_time_bwd(dev, kind, delta, from_uv):
    print("case", kind, delta, from_uv, flush=True)
    spec = _spec(kind)
    cam = _gpu_cam(spec, dev)
    pack = cam.pack.detach().clone().requires_grad_(True)
    g = np.random.default_rng(8)
    if from_uv:
        uv_np = g.uniform(0, 1, (5, 37, 2)).astype(np.float32)
        uv = torch.from_numpy(uv_np).to(dev).requires_grad_(True)
        fn = cam.ext_cls.pixel_time_delta_from_uv if delta else cam.ext_cls.pixel_time_from_uv
        t = fn(pack, uv)
        assert t.shape == (5, 37)
    else:
        fn = cam.ext_cls.pixel_time_delta if delta else cam.ext_cls.pixel_time
        t = fn(pack, W, H)
        assert t.shape == (H, W)
    gr = g.standard_normal(tuple(t.shape)).astype(np.float32)
    (t * torch.from_numpy(gr).to(dev)).sum().backward()
    got = pack.grad.detach().cpu().numpy().reshape(-1)
    if from_uv:
        ref, ref_duv = O.pixel_time_bwd(spec, gr.reshape(-1), uv=uv_np.reshape(-1, 2), delta=delta, prec="f64")
        _close(uv.grad.detach().cpu().numpy().reshape(-1), ref_duv.reshape(-1), "d_uv")
    else:
        ref = O.pixel_time_bwd(spec, gr, W, H, delta=delta, prec="f64")
    _close(got[:21], ref, f"d_pack time {kind}")
    assert np.all(got[21:] == 0)
