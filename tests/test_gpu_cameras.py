"""GPU parity of the distorted-perspective and OpenCV-fisheye camera models against the CPU oracle:
rays with their validity mask, point projection (fixed-point rolling-shutter solve, with and without
camera motion), the unscented-transform projection, the undistort map, and a rendered frame.

Tolerances: rays 2e-5 absolute (five Newton steps of the undistortion in float32 on both sides);
projected uv 1e-4 (the rolling-shutter solve stops at a 1e-4 time residual), depth 1e-5 relative;
UT means / radii 2e-2 pixels; renders 1e-4 absolute. Masks must agree on at least 99.9 % of the
elements (threshold cases can flip on float32 rounding).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from xsimgs_amd import _C, frame, synthetic
from xsimgs_amd.synthetic import CameraSpec
from tests._util import RENDER_ATOL, frac_close, np_, report

pytestmark = pytest.mark.gpu

W, H = 256, 192
MOTION = dict(v=[0.8, -0.2, 0.3], w=[0.3, -0.2, 0.4], rolling=[0.03, 0.01], trigger_time=0.1, pose_time=0.12)


def _spec(kind, moving=True):
    base = synthetic.make_cfg0().cameras[0]
    extra = MOTION if moving else {}
    if kind == "distorted":
        return CameraSpec("distorted", W, H, q=base.q, t=base.t, impl=[0.9, 1.2, 0.5, 0.47],
                          dist=[-0.28, 0.07, 1e-3, -5e-4, 0.01, 0.02, -0.004, 0.001], max_radius=0.9, **extra)
    return CameraSpec("fisheye", W, H, q=base.q, t=base.t, impl=[0.3, 0.4, 0.5, 0.5],
                      dist=[0.03, -0.005, 0.001, -0.0001], **extra)


KINDS = ["distorted", "fisheye"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("world_space,normalized", [(True, True), (False, False), (False, True)])
def test_rays_and_valid(dev, kind, world_space, normalized):
    print("case", kind, world_space, normalized, flush=True)
    spec = _spec(kind)
    cam = frame.make_camera(spec, dev)
    ro, rd, valid = cam.camera_rays(W, H, normalized_rays=normalized, world_space=world_space, return_valid=True)
    rro, rrd, rvalid = O.camera_rays(spec, W, H, world_space, normalized, return_valid=True)
    print(report("ray_d", np_(rd), rrd), "valid", np_(valid).mean(), flush=True)
    assert np.abs(np_(ro) - rro).max() <= 1e-6
    assert np.abs(np_(rd) - rrd).max() <= 2e-5
    assert (np_(valid) == rvalid).mean() >= 0.999


def _points(spec, g, n_rays=4000, n_rand=4000):
    ro, rd = O.camera_rays(spec, W, H, prec="f64")
    idx = g.choice(W * H, n_rays, replace=False)
    on_rays = ro.reshape(-1, 3)[idx] + rd.reshape(-1, 3)[idx] * g.uniform(1.0, 10.0, (n_rays, 1))
    rand = np.asarray(spec.t)[None] + g.uniform(-8, 8, (n_rand, 3))
    return np.concatenate([on_rays, rand]).astype(np.float32)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("moving", [False, True])
@pytest.mark.parametrize("no_jac", [False, True])
def test_projection(dev, kind, moving, no_jac):
    print("case", kind, moving, no_jac, flush=True)
    spec = _spec(kind, moving)
    cam = frame.make_camera(spec, dev)
    pts = _points(spec, np.random.default_rng(1))
    fn = cam.ext_cls.projection_nojac if no_jac else cam.ext_cls.projection
    uvdt, mask = fn(cam.pack, torch.from_numpy(pts).to(dev))
    ruvdt, rmask = O.projection(spec, pts, no_jac=no_jac)
    m, rm = np_(mask), rmask
    agree = (m == rm).mean()
    both = m & rm
    print("mask agree", agree, "valid", int(both.sum()), report("uv", np_(uvdt)[both, :2], ruvdt[both, :2]), flush=True)
    assert agree >= 0.999 and both.sum() > 1000
    np.testing.assert_allclose(np_(uvdt)[both, :2], ruvdt[both, :2], atol=1e-4)
    np.testing.assert_allclose(np_(uvdt)[both, 2], ruvdt[both, 2], rtol=1e-5)
    np.testing.assert_allclose(np_(uvdt)[both, 3], ruvdt[both, 3], atol=1e-5)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("moving", [False, True])
def test_ut_projection(dev, kind, moving):
    print("case", kind, moving, flush=True)
    sc = synthetic.make_cfg0(n=20000)
    spec = _spec(kind, moving)
    cam = frame.make_camera(spec, dev)
    means, scales = sc.means.to(dev), torch.exp(sc.log_scales).to(dev)
    quats, opac = sc.quats.to(dev), torch.sigmoid(sc.opacity_logits).to(dev)
    flags, radii, m2, dep = cam.ext_cls.projection_utgs(cam.pack, means, None, scales, quats, opac, W, H)
    rf, rr, rm, rd = O.project_utgs(spec, sc.means, torch.exp(sc.log_scales), sc.quats,
                                    torch.sigmoid(sc.opacity_logits), W, H)
    f = np_(flags)
    agree = (f == rf).mean()
    both = (f > 0) & (rf > 0)
    print("flags agree", agree, "visible", int(f.sum()), report("means2d", np_(m2)[both], rm[both]),
          report("radii", np_(radii)[both], rr[both]), flush=True)
    assert agree > 0.999 and both.sum() > 500
    assert frac_close(np_(m2)[both], rm[both], 2e-2, 1e-5) > 0.999
    assert frac_close(np_(radii)[both], rr[both], 2e-2, 1e-4) > 0.999
    assert frac_close(np_(dep)[both], rd[both], 1e-5, 1e-5) > 0.999


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("normalized_range", [False, True])
def test_undistort_map(dev, kind, normalized_range):
    spec = _spec(kind)
    cam = frame.make_camera(spec, dev)
    got = cam.undistort_map(W, H, normalized_range=normalized_range)
    ref = O.undistort_map(spec, W, H, normalized_range)
    print(report("map", np_(got), ref), flush=True)
    assert got.shape == (H, W, 2)
    assert np.abs(np_(got) - ref).max() <= 2e-6


def test_undistort_map_only_on_distorted_models():
    assert not hasattr(_C.PerspectiveCamera, "undistort_map")
    assert hasattr(_C.DistortedPerspectiveCamera, "undistort_map")
    assert hasattr(_C.OpenCVFisheyeCamera, "undistort_map")


@pytest.mark.parametrize("kind", KINDS)
def test_render_frame(dev, kind):
    """A whole frame through the distorted model: UT, regular binning, rays and the compositor, checked
    against the oracle's composite of the same binned inputs."""
    print("case", kind, flush=True)
    sc = synthetic.make_cfg0(n=20000, width=W, height=H)
    sc.cameras = [_spec(kind)]
    st = frame.prepare(sc, dev, requires_grad=False)
    out = frame.render_frame(st)
    assert int(out["flatten_ids"].numel()) > 10000
    scales = torch.exp(st.log_scales)
    opac = torch.sigmoid(st.opacity_logits)
    ref = O.eval3d_fwd(np_(st.means), np_(st.quats), np_(scales), np_(out["colors"]), np_(opac), np_(out["ray_o"]),
                       np_(out["ray_d"]), np_(out["offsets"]), np_(out["flatten_ids"]), 16, 16)
    for name, a, b in (("rgb", out["rgb"], ref[0]), ("depth", out["depth"], ref[1]), ("alpha", out["alpha"], ref[2])):
        a = np_(a).reshape(b.shape)
        print(report(name, a, b), "frac", frac_close(a, b, RENDER_ATOL), flush=True)
        assert frac_close(a, b, RENDER_ATOL) > 0.999, name


def test_render_frame_sh_mask_changes_nothing(dev, monkeypatch):
    """render_frame evaluates the SH colours of the Gaussians some tile holds only (the others get
    zeros). The images equal, bit for bit, those of the same frame with every Gaussian's colour (the
    compositor reads no other colour), and so do the colours it reads; the leaf gradients agree to the
    float32 rounding of the compositor's atomic sums, and a Gaussian with no tile gets exact zero SH
    gradients either way."""
    from tests._util import GRAD_ATOL, GRAD_RTOL
    sc = synthetic.make_cfg2(n=200_000)
    runs = []
    for masked in (True, False):
        if not masked:
            monkeypatch.setattr(frame, "REGULAR_TILING", ())  # no regular tiling: colours of all Gaussians
        st = frame.prepare(sc, dev)
        runs.append(frame.render_frame(st, backward=True, grads=(sc.grad_rgb[0], sc.grad_depth[0], sc.grad_alpha[0])))
    a, b = runs
    for k in ("rgb", "depth", "alpha", "flatten_ids", "offsets"):
        assert torch.equal(a[k], b[k]), k
    seen = (a["radii"] > 0).all(-1)
    assert 0 < int(seen.sum()) < seen.numel()
    assert torch.equal(a["colors"][seen], b["colors"][seen])
    assert not a["colors"][~seen].any()
    for k in ("means", "quats", "log_scales", "opacity_logits", "sh"):
        np.testing.assert_allclose(np_(a["grads"][k]), np_(b["grads"][k]), rtol=GRAD_RTOL, atol=GRAD_ATOL,
                                   err_msg=k)
    assert not a["grads"]["sh"][~seen].any() and not b["grads"]["sh"][~seen].any()

@pytest.mark.parametrize("kind", KINDS)
def test_valid_mask_on_folding_lens(dev, kind):
    """Lenses that fold inside the image: the validity masks agree with the oracle and the rays agree
    where the oracle calls them valid (elsewhere the undistortion has no solution)."""
    if kind == "distorted":
        spec = CameraSpec("distorted", W, H, q=[1.0, 0, 0, 0], t=[0, 0, 0], impl=[0.6, 0.8, 0.5, 0.5],
                          dist=[-0.5, 0, 0, 0, 0, 0, 0, 0], max_radius=0.6)
    else:
        spec = CameraSpec("fisheye", W, H, q=[1.0, 0, 0, 0], t=[0, 0, 0], impl=[0.4, 0.5, 0.5, 0.5],
                          dist=[-0.2, 0, 0, 0])
    cam = frame.make_camera(spec, dev)
    _, rd, valid = cam.camera_rays(W, H, world_space=False, normalized_rays=False, return_valid=True)
    _, rrd, rvalid = O.camera_rays(spec, W, H, False, False, return_valid=True)
    v = np_(valid)
    print("valid", v.mean(), "agree", (v == rvalid).mean(), flush=True)
    assert 0.2 < rvalid.mean() < 0.9
    assert (v == rvalid).mean() >= 0.999
    both = v & rvalid
    assert np.abs(np_(rd)[both] - rrd[both]).max() <= 2e-5
