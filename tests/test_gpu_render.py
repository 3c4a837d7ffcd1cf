"""ut_gs_render end to end through autograd (reference render.py:85-187, with rasterize.py:6-72,
rasterize_dynamic.py:10-82 and sh.py:11-42), against the oracle chain.

Leaves are what a trainer optimises: means, log-scales, quaternions, opacity logits, SH coefficients
(and velocities for the dynamic scene). The frame runs the caller's activations (exp, sigmoid) and
spherical_harmonics_fused, then ut_gs_render; torch.autograd.backward takes seeded upstream
gradients. Checked against the oracle:

* the UT projection (judged as in tests/_judge.py), the bool particle mask applied to the radii
  (mask_radii, mask_radii.cu:60-76), binning and tile offsets bit-exact on the GPU's projections;
* ut_gs_render's renders equal the compositor op's on the same binning, and those are judged against
  the oracle's;
* every leaf's gradient against the oracle chain: compositor backward, SH backward for the colour
  gradients (plus its position gradient into the means), and the activations' derivatives
  (log-scales: v_scale * scale; logits: v_opacity * sigmoid * (1 - sigmoid)). The chain is run in
  float32, float64 and float64 with one-ulp moved geometric inputs, and judged as in tests/_judge.py;
  Gaussians no tile lists (masked ones included) must get exactly zero.

Passing the wrong forward inputs to the backward op (scale before quat in, quat before scale out,
eval3d_bwd.cu:406-408) would put a [N, 3] gradient where a [N, 4] one is due, or swap two [N, 3]
ones; either fails here.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from xsimgs_amd import _C, frame, synthetic as S
from xsimgs_amd.rendering import spherical_harmonics_fused, ut_gs_render, ut_gs_tiling
from tests import _judge as J
from tests._util import RENDER_ATOL, frac_close, np_

pytestmark = pytest.mark.gpu

CASES = ["static_sh", "masked", "dynamic"]


def _scene(case):
    g = np.random.default_rng({"static_sh": 600, "masked": 601, "dynamic": 602}[case])
    W, H, n = 96, 64, 3000
    spec = S.pinhole(W, H, 80.0, 80.0, 48.0, 32.0, t=(0.3, -0.2, 0.1))
    deg = 2 if case != "dynamic" else 1
    vel = mask = None
    if case == "dynamic":   # moving rolling-shutter camera and moving Gaussians
        spec.v, spec.w = [1.5, 0.2, -0.4], [0.03, -0.05, 0.1]
        spec.rolling = [0.0, 0.04]
        spec.trigger_time, spec.pose_time = 0.0, 0.02
        vel = g.normal(0, 0.8, (n, 3)).astype(np.float32)
    z = g.uniform(2.0, 15.0, n)
    means = np.stack([g.uniform(-0.65, 0.65, n) * z + 0.3, g.uniform(-0.45, 0.45, n) * z - 0.2, z + 0.1],
                     -1).astype(np.float32)
    log_s = g.normal(-2.6, 0.5, (n, 3)).astype(np.float32)
    quats = g.normal(0, 1, (n, 4)).astype(np.float32)   # not normalised: the kernels normalise
    logits = g.normal(0.0, 1.5, n).astype(np.float32)
    sh = np.concatenate([g.normal(0, 0.3, (n, 1, 3)), g.normal(0, 0.05, (n, (deg + 1) ** 2 - 1, 3))], 1)
    sh = sh.astype(np.float32)
    if case == "masked":
        mask = g.random(n) > 0.3
    grads = [(g.normal(0, 1e-3, s)).astype(np.float32) for s in ((H, W, 3), (H, W), (H, W))]
    return dict(spec=spec, W=W, H=H, deg=deg, means=means, log_s=log_s, quats=quats, logits=logits, sh=sh,
                vel=vel, mask=mask, grads=grads)


def _chain(prec, d, deg, origin, tsx, tsy):
    """The oracle's gradients of every leaf, given the GPU's forward state."""
    g = O.eval3d_bwd(d["means"], d["quats"], d["scales"], d["colors"], d["opac"], d["ro"], d["rd"], d["off"], d["fl"],
                     d["alpha"], d["last"], d["v_rgb"], d["v_d"], d["v_a"], tsx, tsy, velocity=d.get("vel"),
                     ray_time_delta=d.get("rtd"), prec=prec)
    d_co, _, d_pos, _ = O.sh_bwd(deg, origin, d["means"], d["sh"], g["v_colors"], prec=prec)
    out = dict(means=g["v_means"] + d_pos, quats=g["v_quats"], log_scales=g["v_scales"] * d["scales"],
               opacity_logits=g["v_opacity"] * d["opac"] * (1.0 - d["opac"]), sh=d_co)
    if d.get("vel") is not None:
        out["velocity"] = g["v_velocity"]
    return out


@pytest.mark.parametrize("case", CASES)
def test_ut_gs_render_autograd(dev, case):
    print("case", case, flush=True)
    s = _scene(case)
    spec, W, H, deg = s["spec"], s["W"], s["H"], s["deg"]
    tsx = tsy = 16
    L = lambda a: None if a is None else torch.from_numpy(a).to(dev).requires_grad_(True)
    means, log_s, quats, logits, sh, vel = (L(s[k]) for k in ("means", "log_s", "quats", "logits", "sh", "vel"))
    mask = None if s["mask"] is None else torch.from_numpy(s["mask"]).to(dev)
    cam = frame.make_camera(spec, dev)
    origin = cam.pose.t
    scales = torch.exp(log_s)
    opac = torch.sigmoid(logits)
    colors = spherical_harmonics_fused(sh, means, origin, deg)
    rgb, depth, alpha, meta = ut_gs_render(cam, means, scales, quats, opac, W, H, colors=colors, points_velocity=vel,
                                           packed_particle_mask=mask, tile_size_x=tsx, tile_size_y=tsy)
    g_rgb, g_d, g_a = (torch.from_numpy(x).to(dev) for x in s["grads"])
    torch.autograd.backward([rgb, depth, alpha], [g_rgb, g_d, g_a])
    got = dict(means=means.grad, quats=quats.grad, log_scales=log_s.grad, opacity_logits=logits.grad, sh=sh.grad)
    if vel is not None:
        got["velocity"] = vel.grad
    for k, v in got.items():
        assert v is not None and torch.isfinite(v).all(), k

    with torch.no_grad():
        hs, ho, hc = np_(scales), np_(opac), np_(colors)
        hm, hq = s["means"], s["quats"]
        # colours
        ref_col = O.sh_fwd(deg, np_(origin), hm, s["sh"])
        assert frac_close(hc, ref_col, RENDER_ATOL) == 1.0
        # UT (unmasked) and the bool mask on its radii
        proj = cam.ut_gs_projection(means, scales, quats, W, H, points_velocity=vel, opacity=opac)
        J.judge_ut(proj, spec, hm, hs, hq, ho, W, H, label=case, vel=s["vel"])
        tiles = ut_gs_tiling(cam, means, scales, quats, W, H, points_velocity=vel, opacity=opac,
                             packed_particle_mask=mask, tile_size_x=tsx, tile_size_y=tsy)
        radii = np_(proj[1]).copy()
        if s["mask"] is not None:
            radii = O.mask_radii(radii, mask=s["mask"])
            assert int((~s["mask"] & (np_(proj[1]) > 0).all(-1)).sum()) > 100   # the mask removes visible ones
        assert np.array_equal(np_(tiles["radii"]), radii)
        assert np.array_equal(np_(meta["radii"]), radii)
        # binning on the (masked) projections
        tpg, ids, fl = O.isect_regular(np_(proj[2]), radii, np_(proj[3]), W, H, tsx, tsy)
        ntx, nty = (W + tsx - 1) // tsx, (H + tsy - 1) // tsy
        off = O.offset_encode(ids, ntx, nty)
        assert np.array_equal(np_(tiles["flatten_ids"]), fl)
        assert np.array_equal(np_(tiles["isect_offsets"]), off)
        if s["mask"] is not None:
            assert not np.any(np.isin(fl, np.nonzero(~s["mask"])[0]))
        # renders: ut_gs_render's equal the compositor op's, which are judged against the oracle
        ro, rd = cam.camera_rays(W, H)
        rtd = cam.image_time_delta(ro) if vel is not None else None
        T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        if vel is None:
            direct = _C.rasterize_eval3d_fwd(means, quats, scales, colors.unsqueeze(0), opac.view(1, -1), W, H, tsx,
                                             tsy, ro, rd, T(off), T(fl))
        else:
            direct = _C.rasterize_eval3d_dynamic_fwd(means, vel, quats, scales, colors.unsqueeze(0), opac.view(1, -1),
                                                     W, H, tsx, tsy, ro, rd, rtd, T(off), T(fl))
        for a, b in zip((rgb, depth, alpha), direct[:3]):
            assert torch.equal(a, b)
        hro, hrd = np_(ro), np_(rd)
        hrtd = None if rtd is None else np_(rtd)[..., 0]
        fwd = [np_(x) for x in direct]
        inp = dict(means=hm, quats=hq, scales=hs, opac=ho, colors=hc, ro=hro, rd=hrd, vel=s["vel"], rtd=hrtd)
        ref32 = O.eval3d_fwd(hm, hq, hs, hc, ho, hro, hrd, off, fl, tsx, tsy, velocity=s["vel"], ray_time_delta=hrtd)
        J.judge_renders(fwd, ref32, inp, off, fl, tsx, tsy, label=case)

    # gradients of every leaf against the oracle chain
    v_rgb, v_d, v_a = s["grads"]
    base = dict(means=hm, quats=hq, scales=hs, opac=ho, colors=hc, ro=hro, rd=hrd, vel=s["vel"], rtd=hrtd, off=off,
                fl=fl, alpha=fwd[2], last=fwd[3], v_rgb=v_rgb, v_d=v_d, v_a=v_a, sh=s["sh"])
    o = np_(origin)
    r32 = _chain("f32", base, deg, o, tsx, tsy)
    r64 = _chain("f64", base, deg, o, tsx, tsy)
    rng = np.random.default_rng(7)
    moved = []
    for _ in range(2):
        d = dict(base)
        for k in ("means", "quats", "scales", "ro", "rd", "vel", "rtd"):
            if d.get(k) is not None:
                d[k] = J.move_ulp(d[k], rng)
        moved.append(_chain("f64", d, deg, o, tsx, tsy))
    rows = np.unique(fl)
    got_n = {k: np_(v).reshape(v.shape[0], -1) for k, v in got.items()}
    flat = lambda r: {k: v.reshape(v.shape[0], -1) for k, v in r.items()}
    J.judge_grads(got_n, (flat(r32), flat(r64), [flat(m) for m in moved]), rows, label=case)
