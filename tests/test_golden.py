"""Committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture (guards the checker itself).
GPU: every stage of the HIP path, fed the fixture's upstream values, reproduces the fixture:
binning, sorted keys, flatten ids and tile ranges bit-exact; projections, colours and renders
within 1e-4 absolute; gradients within 1e-3 relative with a 1e-5 absolute floor.
"""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from xsimgs_amd import synthetic as S
from tests import _judge as J
from tests._util import GRAD_ATOL, GRAD_RTOL, RENDER_ATOL, frac_close, np_, report

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = ["pinhole_sh", "lidar_phm", "spherical", "dynamic"]
KIND_NAMES = {0: "pinhole", 1: "spherical", 2: "lidar"}


def load(name):
    with np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False) as z:
        f = {k: z[k] for k in z.files}
    w, h = (int(x) for x in f["cam_size"])
    spec = S.CameraSpec(KIND_NAMES[int(f["cam_kind"])], w, h, f["cam_q"].tolist(), f["cam_t"].tolist(),
                        f["cam_impl"].tolist(), v=f["cam_v"].tolist(), w=f["cam_w"].tolist(),
                        rolling=f["cam_rolling"].tolist(), trigger_time=float(f["cam_times"][0]),
                        pose_time=float(f["cam_times"][1]),
                        beam_v=torch.from_numpy(f["cam_beam_v"]) if "cam_beam_v" in f else None)
    return spec, f


GRAD_KEYS = ["v_means", "v_quats", "v_scales", "v_opacity", "v_colors", "v_ray_o", "v_ray_d"]


# ------------------------------------------------------------------ CPU: the oracle reproduces the fixtures
@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_fixture(name):
    spec, f = load(name)
    W, H = spec.width, spec.height
    tsx, tsy = (int(x) for x in f["tile"])
    vel = f.get("velocity")
    phm = name in ("lidar_phm", "spherical")
    flags, radii, m2, dep = O.project_utgs(spec, f["means"], f["scales"], f["quats"], f["opacity"], W, H, vel=vel,
                                           phm=phm)
    assert np.array_equal(flags, f["ut_flags"])
    for a, k in ((radii, "radii"), (m2, "means2d"), (dep, "depths")):
        assert np.allclose(a, f[k], rtol=1e-6, atol=1e-6), k
    if spec.kind == "pinhole":
        tpg, ids, fl = O.isect_regular(f["means2d"], f["radii"], f["depths"], W, H, tsx, tsy)
    else:
        tpg, ids, fl = O.isect_spherical_family(spec.kind, spec, f["means"], f["scales"], f["quats"], f["opacity"],
                                                f["ut_flags"], f["means2d"], f["radii"], f["depths"], tsx, tsy, W, H,
                                                elev=f.get("elev"))
    assert np.array_equal(tpg, f["tiles_per_gauss"])
    assert np.array_equal(ids, f["isect_ids"]) and np.array_equal(fl, f["flatten_ids"])
    nth, ntw = f["offsets"].shape
    assert np.array_equal(O.offset_encode(ids, ntw, nth), f["offsets"])
    ro, rd = O.camera_rays(spec, W, H)
    assert np.array_equal(ro, f["ray_o"]) and np.array_equal(rd, f["ray_d"])
    rtd = f.get("ray_time_delta")
    out = O.eval3d_fwd(f["means"], f["quats"], f["scales"], f["colors"], f["opacity"], f["ray_o"], f["ray_d"],
                       f["offsets"], f["flatten_ids"], tsx, tsy, velocity=vel, ray_time_delta=rtd)
    for a, k in zip(out, ("rgb", "depth", "alpha", "last_ids")):
        assert np.array_equal(a, f[k]), k
    gr = O.eval3d_bwd(f["means"], f["quats"], f["scales"], f["colors"], f["opacity"], f["ray_o"], f["ray_d"],
                      f["offsets"], f["flatten_ids"], f["alpha"], f["last_ids"], f["v_rgb"], f["v_depth"],
                      f["v_alpha"], tsx, tsy, velocity=vel, ray_time_delta=rtd)
    for k, v in gr.items():   # the threaded backward sums in a varying order: float32 rounding only
        ref = f["g_" + k]
        assert np.allclose(v, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max()), k
    # the fixtures exercise what they are meant to
    assert (f["alpha"] > 0.5).mean() > 0.2
    if phm:
        assert (f["ut_flags"] == 2).sum() > 5


# ------------------------------------------------------------------ GPU: the HIP path reproduces the fixtures
def _t(a, dev):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _check(name, got, ref, atol, rtol=0.0, min_frac=1.0):
    fc = frac_close(np_(got), ref, atol, rtol)
    print(report(name, np_(got), ref), "frac", fc, flush=True)
    assert np_(got).shape == ref.shape, name
    assert fc >= min_frac, name


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_hip_path_reproduces_fixture(dev, name):
    from xsimgs_amd import _C, frame
    print("golden case", name, flush=True)
    spec, f = load(name)
    W, H = spec.width, spec.height
    tsx, tsy = (int(x) for x in f["tile"])
    T = lambda k: _t(f[k], dev) if k in f else None
    cam = frame.make_camera(spec, dev)
    pack = cam.pack
    means, scales, quats, opac, vel = T("means"), T("scales"), T("quats"), T("opacity"), T("velocity")

    # SH colours and their backward
    if "sh" in f:
        deg = int(f["sh_degree"])
        origin = _t(f["cam_t"], dev)
        colors = _C.spherical_harmonics_fused_fwd(deg, origin, means, T("sh"), None, False)
        _check("sh colors", colors, f["colors"], RENDER_ATOL)
        dco, _, dpos, dori = _C.spherical_harmonics_fused_bwd(deg, origin, means, T("sh"), None, False,
                                                              T("g_v_colors"))
        _check("sh d_coeffs", dco, f["sh_d_coeffs"], GRAD_ATOL, GRAD_RTOL)
        _check("sh d_positions", dpos, f["sh_d_positions"], GRAD_ATOL, GRAD_RTOL)
        _check("sh d_origin", dori, f["sh_d_origin"], GRAD_ATOL, GRAD_RTOL)

    # point projection (rolling shutter, moving camera and points)
    if "proj_uvdt" in f:
        uvdt, mask = cam.ext_cls.projection(pack, means, vel)
        m = np_(mask).astype(bool)
        # a validity disagreement only where float32 does not decide it: the f64 landing point within
        # 1e-5 of the image's [0, 1] bounds (the last test of projection_kernels.h:255 and the caller's
        # in-image check), else the mask must be f64's
        dis = np.nonzero(m != f["proj_mask"])[0]
        if dis.size:
            u64, m64 = O.projection(spec, f["means"], vel=f.get("velocity"), prec="f64")
            uv = u64[dis, :2]
            near = (np.minimum(np.abs(uv), np.abs(uv - 1.0)) < 1e-5).any(-1)
            print("projection mask disagreements", dis.size, "near the image bounds", int(near.sum()), flush=True)
            assert np.all(near | (m[dis] == m64[dis].astype(bool))), dis[~near]
        both = m & f["proj_mask"]
        _check("projection uvdt", np_(uvdt)[both], f["proj_uvdt"][both], 1e-5, 1e-5)
        rtd = cam.ext_cls.pixel_time_delta(pack, W, H)
        _check("pixel time delta", rtd, f["ray_time_delta"], 1e-6)

    # UT projection
    phm = name in ("lidar_phm", "spherical")
    vel_np = f.get("velocity")
    proj = cam.ext_cls.projection_utgs_phm if phm else cam.ext_cls.projection_utgs
    flags, radii, m2, dep = proj(pack, means, vel, scales, quats, opac, W, H)
    agree = (np_(flags) == f["ut_flags"]).mean()
    print("ut flags agree", agree, flush=True)
    J.judge_ut((flags, radii, m2, dep), spec, f["means"], f["scales"], f["quats"], f["opacity"], W, H, phm=phm,
               label=name, vel=vel_np)

    # binning from the fixture's projections: bit-exact
    m2f, rf, df, ff = T("means2d"), T("radii"), T("depths"), T("ut_flags")

    def binning(**kw):
        if spec.kind == "pinhole":
            return _C.isect_regular_tiles(m2f, rf, df, W, H, tsx, tsy, **kw)
        if spec.kind == "lidar":
            return _C.isect_lidar_tiles(pack, means, vel, scales, quats, opac, ff, m2f, rf, df, T("elev"), tsx, W, H,
                                        **kw)
        return _C.isect_spherical_tiles(pack, means, vel, scales, quats, opac, ff, m2f, rf, df, tsx, tsy, W, H, **kw)

    tpg, ids, fl = binning()
    if spec.kind == "pinhole" and "isect_ids_unsorted" in f:
        _, ids_u, fl_u = binning(sort=False)
        assert np.array_equal(np_(ids_u), f["isect_ids_unsorted"])
        assert np.array_equal(np_(fl_u), f["flatten_ids_unsorted"])
    nth, ntw = f["offsets"].shape
    und = None
    if spec.kind != "pinhole":
        und = O.isect_spherical_family(spec.kind, spec, f["means"], f["scales"], f["quats"], f["opacity"],
                                       f["ut_flags"], f["means2d"], f["radii"], f["depths"], tsx, tsy, W, H,
                                       elev=f.get("elev"), vel=vel_np, seam_margins=True) < 1.0
    fs = lambda g, t: J.first_span_member(spec.kind, spec, g, t, f["means2d"], f["radii"], W, H, tsx, tsy,
                                          f.get("elev"))
    J.check_binning(spec.kind, (np_(tpg), np_(ids), np_(fl)), (f["tiles_per_gauss"], f["isect_ids"],
                    f["flatten_ids"]), f["ut_flags"], f["depths"], ntw * nth, name, und, fs)
    off = _C.isect_offset_encode(ids, ntw, nth)
    assert np.array_equal(np_(off), O.offset_encode(np_(ids), ntw, nth))
    if np.array_equal(np_(tpg), f["tiles_per_gauss"]):
        assert np.array_equal(np_(off), f["offsets"])
    # the sorted fill's own tile offsets (extension, what ut_gs_tiling uses) are the encoder's
    fill_off = torch.full((nth, ntw), -7, dtype=torch.int32, device=dev)
    _, ids2, _ = binning(tile_offsets=fill_off)
    assert np.array_equal(np_(ids2), np_(ids))
    assert np.array_equal(np_(fill_off), np_(off))

    # rays
    ro, rd = cam.camera_rays(W, H)
    _check("ray_o", ro, f["ray_o"], 2e-6)
    _check("ray_d", rd, f["ray_d"], 2e-6)

    # composite forward and backward from the fixture's rays, ranges and colours
    colors, ro, rd, off, fl = T("colors"), T("ray_o"), T("ray_d"), T("offsets"), T("flatten_ids")
    if vel is not None:
        rgb, depth, alpha, last = _C.rasterize_eval3d_dynamic_fwd(means, vel, quats, scales, colors.unsqueeze(0),
                                                                  opac.view(1, -1), W, H, tsx, tsy, ro, rd,
                                                                  T("ray_time_delta"), off, fl)
    else:
        rgb, depth, alpha, last = _C.rasterize_eval3d_fwd(means, quats, scales, colors.unsqueeze(0), opac.view(1, -1),
                                                          W, H, tsx, tsy, ro, rd, off, fl)
    # renders against the fixture (the f32 oracle's): every pixel outside 1e-4 or with another last id
    # undetermined in float32 or right against f64 (tests/_judge.py)
    rtd_np = f["ray_time_delta"] if vel is not None else None
    inp = dict(means=f["means"], quats=f["quats"], scales=f["scales"], opac=f["opacity"], colors=f["colors"],
               ro=f["ray_o"], rd=f["ray_d"], vel=f.get("velocity"), rtd=rtd_np)
    J.judge_renders([np_(rgb), np_(depth), np_(alpha), np_(last)], (f["rgb"], f["depth"], f["alpha"], f["last_ids"]),
                    inp, f["offsets"], f["flatten_ids"], tsx, tsy, label=name)
    args = dict(render_alpha=T("alpha"), last_ids=T("last_ids"), v_render_colors=T("v_rgb"),
                v_render_depth=T("v_depth"), v_render_alpha=T("v_alpha"))
    if vel is not None:
        grads = _C.rasterize_eval3d_dynamic_bwd(means, vel, scales, quats, opac, colors, ro, rd, T("ray_time_delta"),
                                                tsx, tsy, off, fl, **args)
        keys = ["v_means", "v_velocity", "v_quats", "v_scales", "v_opacity", "v_colors", "v_ray_o", "v_ray_d",
                "v_time_delta"]          # eval3d_dynamic_bwd.cu:427
    else:
        grads = _C.rasterize_eval3d_bwd(means, scales, quats, opac, colors, ro, rd, tsx, tsy, off, fl, **args)
        keys = GRAD_KEYS
    assert len(grads) == len(keys)
    got = dict(zip(keys, grads))
    # gradients judged against f64 on every Gaussian and pixel float32 determines (tests/_judge.py),
    # from the fixture's alpha and last ids as the kernel was given them; the fixture's own gradients
    # are the f32 oracle's (test_oracle_reproduces_fixture)
    refs = J.bwd_runs(inp, f["offsets"], f["flatten_ids"], f["alpha"], f["last_ids"], f["v_rgb"], f["v_depth"],
                      f["v_alpha"], tsx, tsy, None)
    gk = [k for k in ("v_means", "v_quats", "v_scales", "v_opacity", "v_colors", "v_velocity") if k in got]
    J.judge_grads({k: got[k] for k in gk}, refs, np.unique(f["flatten_ids"]), label=name)
    pk = [k for k in ("v_ray_o", "v_ray_d", "v_time_delta") if k in got]
    J.judge_pixel_grads({k: got[k] for k in pk}, refs, np.ones(f["alpha"].shape, bool), label=name)


@pytest.mark.gpu
@pytest.mark.parametrize("table", ["unsorted", "long"])
def test_lidar_elevation_tables(dev, table):
    """The lidar count pass finds each Gaussian's elevation rows as find_bounds_increasing scans them
    (phm_lidar_tiling.cu:35-60): by bisection when the table is non-decreasing and fits in LDS (the
    golden lidar scene and cfg3 take that path), else by the same linear scan. Two boundaries swapped
    (not non-decreasing) and a table of 1100 boundaries (more than the 1024 kept in LDS) take the scan;
    both must bin as the oracle does with the same table."""
    from xsimgs_amd import _C, frame
    print("elevation table", table, flush=True)
    spec, f = load("lidar_phm")
    W, H = spec.width, spec.height
    tsx, tsy = (int(x) for x in f["tile"])
    elev = f["elev"].astype(np.float32).copy()
    if table == "unsorted":
        k = elev.size // 2
        elev[k], elev[k + 1] = elev[k + 1], elev[k]
        assert np.any(np.diff(elev) < 0)
    else:
        x = np.linspace(0.0, elev.size - 1.0, 1100)
        elev = np.interp(x, np.arange(elev.size), elev.astype(np.float64)).astype(np.float32)
        assert elev.size > 1024 and np.all(np.diff(elev) >= 0)
    T = lambda k: _t(f[k], dev) if k in f else None
    cam = frame.make_camera(spec, dev)
    vel_np = f.get("velocity")
    tpg, ids, fl = _C.isect_lidar_tiles(cam.pack, T("means"), T("velocity"), T("scales"), T("quats"), T("opacity"),
                                        T("ut_flags"), T("means2d"), T("radii"), T("depths"), _t(elev, dev), tsx, W,
                                        H)
    args = (spec.kind, spec, f["means"], f["scales"], f["quats"], f["opacity"], f["ut_flags"], f["means2d"],
            f["radii"], f["depths"], tsx, tsy, W, H)
    ref = O.isect_spherical_family(*args, elev=elev, vel=vel_np)
    und = O.isect_spherical_family(*args, elev=elev, vel=vel_np, seam_margins=True) < 1.0
    ntw = (W + tsx - 1) // tsx
    fs = lambda g, t: J.first_span_member(spec.kind, spec, g, t, f["means2d"], f["radii"], W, H, tsx, tsy, elev)
    J.check_binning(spec.kind, (np_(tpg), np_(ids), np_(fl)), ref, f["ut_flags"], f["depths"], ntw * elev.size,
                    f"lidar_phm {table} elevation table", und, fs)
