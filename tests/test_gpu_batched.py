"""Batched cameras (an extension of this build): C cameras over one scene composited in one launch per
pass (rasterize_eval3d_{fwd,bwd}_batched) and the rig frame built on it (frame.render_rig).

The reference composites one camera per call (eval3d_fwd.cu:248-316 allocates one image), so the
oracle for a batched call is the single-camera path this suite already judges against the CPU
oracle: every camera's slice of a batched call must equal a single-camera call on that camera's
binning.

* forward: renders, depth and alpha bit-exact; last ids equal the single call's shifted by the
  camera's first intersection (0 where no Gaussian was composited); the pair counts add up exactly;
* backward: the per-Gaussian gradients equal the sum of the single calls' and the per-camera colour
  and ray gradients equal each call's own, up to the order of the float atomics (1e-5 of the
  largest value of each gradient, 1e-4 relative); colours shared by every camera get the sum over
  the cameras;
* the batched binning equals the single-camera binning of every camera with the camera id added
  above the tile bits (its own bit-exact test against the oracle is test_isect_regular_tile_shapes);
* render_rig on the cfg4 rig (six co-located cameras, one SH evaluation) against render_frame called
  once per camera: images bit-exact and every leaf's accumulated gradient within the same bound.
"""
import numpy as np
import pytest
import torch

from xsimgs_amd import _C, frame, synthetic as S
from xsimgs_amd.rendering import spherical_harmonics_fused
from tests._util import np_

pytestmark = pytest.mark.gpu

ATOL_FRAC = 1e-5   # of the largest |value| of the gradient
RTOL = 1e-4


def _close(name, got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (name, got.shape, want.shape)
    scale = max(float(np.abs(want).max()) if want.size else 0.0, 1e-30)
    bad = np.abs(got - want) > ATOL_FRAC * scale + RTOL * np.abs(want)
    assert not bad.any(), (f"{name}: {int(bad.sum())} of {bad.size} differ, max|d| "
                           f"{np.abs(got - want).max():.3e}, max|want| {scale:.3e}")


def _rig(case, dev):
    g = np.random.default_rng({"per_camera": 700, "shared": 701, "dynamic": 702}[case])
    W, H, n, C = 200, 136, 30_000, 4
    specs = []
    for i in range(C):
        yaw = 2.0 * np.pi * i / C
        q = S._quat_mul(S._axis_angle_quat([0.0, 0.0, 1.0], yaw), [0.5, -0.5, 0.5, -0.5])
        t = (0.0, 0.0, 0.0) if case == "shared" else (0.2 * i, -0.1 * i, 0.05 * i)
        sp = S.pinhole(W, H, 150.0, 150.0, W / 2, H / 2, q=q, t=t)
        if case == "dynamic":   # moving rolling-shutter cameras
            sp.v, sp.w = [1.0, 0.3, -0.2], [0.02, -0.03, 0.05]
            sp.rolling = [0.0, 0.03]
            sp.pose_time = 0.015
        specs.append(sp)
    r = g.uniform(3.0, 25.0, n)
    az = g.uniform(0.0, 2.0 * np.pi, n)
    means = np.stack([r * np.cos(az), r * np.sin(az), g.uniform(-3.0, 3.0, n)], -1).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
    d = dict(W=W, H=H, n=n, C=C, specs=specs, cams=[frame.make_camera(sp, dev) for sp in specs],
             means=T(means), scales=T(np.exp(g.normal(-2.2, 0.5, (n, 3)))), quats=T(g.normal(0, 1, (n, 4))),
             opac=T(1.0 / (1.0 + np.exp(-g.normal(0.5, 1.5, n)))), sh=T(g.normal(0, 0.3, (n, 9, 3))),
             vel=T(g.normal(0, 0.5, (n, 3))) if case == "dynamic" else None)
    d["grads"] = [T(g.normal(0, 1e-3, s)) for s in ((C, H, W, 3), (C, H, W), (C, H, W))]
    return d


@pytest.mark.parametrize("case", ["per_camera", "shared", "dynamic"])
def test_batched_compositor_matches_single(dev, case):
    print("case", case, flush=True)
    d = _rig(case, dev)
    W, H, C, n = d["W"], d["H"], d["C"], d["n"]
    tsx, tsy = 16, 16
    ntx, nty = (W + tsx - 1) // tsx, (H + tsy - 1) // tsy
    means, scales, quats, opac, vel = d["means"], d["scales"], d["quats"], d["opac"], d["vel"]
    proj, rays, cols, rtds, single_bins = [], [], [], [], []
    for cam in d["cams"]:
        with cam._freeze_ctx():
            fl_, radii, m2, dep = cam.ut_gs_projection(means, scales, quats, W, H, points_velocity=vel, opacity=opac)
            ro, rd = cam.camera_rays(W, H)
        proj.append((radii, m2, dep))
        rays.append((ro, rd))
        cols.append(spherical_harmonics_fused(d["sh"], means, cam.pose.t, 2))
        rtds.append(cam.image_time_delta(ro)[..., 0].contiguous() if vel is not None else None)
        off = torch.empty((nty, ntx), dtype=torch.int32, device=dev)
        _, ids, fl = _C.isect_regular_tiles(radii=radii, means2d=m2, depth=dep, img_width=W, img_height=H,
                                            tile_size_x=tsx, tile_size_y=tsy, tile_offsets=off)
        single_bins.append((ids, fl, off))

    # batched binning = the single binnings with the camera id above the tile bits
    boff = torch.empty((C, nty, ntx), dtype=torch.int32, device=dev)
    stack = lambda k: torch.stack([p[k] for p in proj])
    _, bids, bfl = _C.isect_regular_tiles_batched(stack(1), stack(0), stack(2), W, H, tsx, tsy, tile_offsets=boff)
    tile_bits = int(ntx * nty).bit_length()   # floor(log2(n_tiles)) + 1, regular_tiling.cu:96-97
    starts = []
    pos = 0
    for ci, (ids, fl, off) in enumerate(single_bins):
        k = ids.numel()
        starts.append(pos)
        assert torch.equal(bids[pos:pos + k], ids + (ci << (32 + tile_bits))), ci
        assert torch.equal(bfl[pos:pos + k], fl + ci * n), ci
        assert torch.equal(boff[ci], off + pos), ci
        pos += k
    assert pos == bids.numel()

    shared = case == "shared"
    colors = cols[0] if shared else torch.stack(cols)
    if shared:
        for c in cols[1:]:
            assert torch.equal(c, cols[0])
    ro_b = torch.stack([r[0] for r in rays])
    rd_b = torch.stack([r[1] for r in rays])
    rtd_b = torch.stack(rtds) if vel is not None else None
    pairs_b = torch.zeros(2, dtype=torch.int64, device=dev)
    out_b = _C.rasterize_eval3d_fwd_batched(means, quats, scales, colors, opac, W, H, tsx, tsy, ro_b, rd_b, boff,
                                            bfl, velocity=vel, ray_time_delta=rtd_b, pair_counts=pairs_b)
    assert out_b[0].shape == (C, H, W, 3) and out_b[3].shape == (C, H, W)
    pairs_s = torch.zeros(2, dtype=torch.int64, device=dev)
    singles = []
    for ci in range(C):
        ids, fl, off = single_bins[ci]
        ro, rd = rays[ci]
        if vel is None:
            o = _C.rasterize_eval3d_fwd(means, quats, scales, cols[ci].unsqueeze(0), opac.view(1, -1), W, H, tsx,
                                        tsy, ro, rd, off, fl, pair_counts=pairs_s)
        else:
            o = _C.rasterize_eval3d_dynamic_fwd(means, vel, quats, scales, cols[ci].unsqueeze(0), opac.view(1, -1),
                                                W, H, tsx, tsy, ro, rd, rtds[ci], off, fl, pair_counts=pairs_s)
        singles.append(o)
        for k in range(3):
            assert torch.equal(out_b[k][ci], o[k]), (ci, k)
        took = o[2] > 0
        want_last = torch.where(took, o[3] + starts[ci], torch.zeros_like(o[3]))
        assert torch.equal(torch.where(took, out_b[3][ci], torch.zeros_like(o[3])), want_last), ci
        assert int((out_b[3][ci][~took] != 0).sum()) == 0, ci
    assert torch.equal(pairs_b, pairs_s)
    assert float(out_b[2].max()) > 0.5   # the scene covers the images

    # backward
    v_rgb, v_d, v_a = d["grads"]
    gb = _C.rasterize_eval3d_bwd_batched(means, scales, quats, opac, colors, ro_b, rd_b, tsx, tsy, boff, bfl,
                                         out_b[2], out_b[3], v_rgb, v_d, v_a, velocity=vel, ray_time_delta=rtd_b)
    acc = None
    per_cam = []
    for ci in range(C):
        ids, fl, off = single_bins[ci]
        ro, rd = rays[ci]
        o = singles[ci]
        if vel is None:
            gs = _C.rasterize_eval3d_bwd(means, scales, quats, opac, cols[ci], ro, rd, tsx, tsy, off, fl, o[2], o[3],
                                         v_rgb[ci], v_d[ci], v_a[ci])
            gs = list(gs[:4]) + [gs[4], gs[5], gs[6], None, None]
        else:
            r = _C.rasterize_eval3d_dynamic_bwd(means, vel, scales, quats, opac, cols[ci], ro, rd, rtds[ci], tsx, tsy,
                                                off, fl, o[2], o[3], v_rgb[ci], v_d[ci], v_a[ci])
            gs = [r[0], r[2], r[3], r[4], r[5], r[6], r[7], r[1], r[8]]
        per_cam.append(gs)
        acc = [np_(x).astype(np.float64) for x in gs[:4]] if acc is None else \
            [a + np_(x) for a, x in zip(acc, gs[:4])]
    for k, name in enumerate(("v_means", "v_quats", "v_scales", "v_opacities")):
        _close(f"{case} {name}", np_(gb[k]), acc[k])
    if shared:
        _close(f"{case} v_colors", np_(gb[4]), sum(np_(g[4]).astype(np.float64) for g in per_cam))
    else:
        for ci in range(C):
            _close(f"{case} v_colors cam {ci}", np_(gb[4][ci]), np_(per_cam[ci][4]))
    for ci in range(C):
        _close(f"{case} v_ray_o cam {ci}", np_(gb[5][ci]), np_(per_cam[ci][5]))
        _close(f"{case} v_ray_d cam {ci}", np_(gb[6][ci]), np_(per_cam[ci][6]))
    if vel is not None:
        _close(f"{case} v_velocity", np_(gb[7]), sum(np_(g[7]).astype(np.float64) for g in per_cam))
        for ci in range(C):
            _close(f"{case} v_time_delta cam {ci}", np_(gb[8][ci]), np_(per_cam[ci][8]))


def test_batched_compositor_rejects_bad_shapes(dev):
    d = _rig("shared", dev)
    W, H, n = d["W"], d["H"], d["n"]
    ro = torch.zeros((2, H, W, 3), device=dev)
    off = torch.zeros((2, 9, 13), dtype=torch.int32, device=dev)
    fl = torch.zeros(0, dtype=torch.int32, device=dev)
    cols = torch.zeros((3, n, 3), device=dev)   # three colour sets for two cameras
    with pytest.raises(RuntimeError, match="colors must be"):
        _C.rasterize_eval3d_fwd_batched(d["means"], d["quats"], d["scales"], cols, d["opac"], W, H, 16, 16, ro, ro,
                                        off, fl)
    with pytest.raises(RuntimeError, match="tile_offsets"):
        _C.rasterize_eval3d_fwd_batched(d["means"], d["quats"], d["scales"], cols[0], d["opac"], W, H, 16, 16, ro, ro,
                                        off[0], fl)


@pytest.mark.parametrize("size", ["200k", "full"])
def test_render_rig_matches_camera_loop(dev, size):
    """The cfg4 rig (six co-located cameras): render_rig (the frame the cfg4 benchmark line times) against
    render_frame per camera (the reference caller's loop, camera.h:58-59), forward and every leaf's
    gradient, with 200k Gaussians and at the benchmark's full size (4M Gaussians in 2000 blobs: 24M
    camera instances and ~33M intersections in one batched binning, which takes the size-dependent
    paths: the large pre-order tiles and the single-pass rig row sort). Each camera's slice of the
    batched binning (its tile offsets, its flatten ids less the camera's first row) equals that camera's
    own binning bit for bit."""
    sc = S.make_cfg4(seed=3, n=200_000, n_blobs=300) if size == "200k" else S.make_cfg4()
    print("rig", size, sc.n, "Gaussians", flush=True)
    st = frame.prepare(sc, dev)
    assert frame.rig_batchable(st) and frame.rig_shares_origin(st)
    C = len(sc.cameras)
    frame.zero_grads(st)
    grads = [torch.stack([getattr(sc, k)[i] for i in range(C)]) for k in ("grad_rgb", "grad_depth", "grad_alpha")]
    rig = frame.render_rig(st, backward=True, grads=grads)
    got = {k: np_(v).astype(np.float64) for k, v in rig["grads"].items() if v is not None}
    r_off = np_(rig["offsets"]).astype(np.int64)
    r_fl = np_(rig["flatten_ids"])
    n_rig = r_fl.size
    frame.zero_grads(st)
    total = 0
    for ci in range(C):
        o = frame.render_frame(st, backward=True, cam_index=ci,
                               grads=(sc.grad_rgb[ci], sc.grad_depth[ci], sc.grad_alpha[ci]))
        for k in ("rgb", "depth", "alpha"):
            assert torch.equal(rig[k][ci].detach(), o[k].detach()), (ci, k)
        off1, fl1 = np_(o["offsets"]).astype(np.int64), np_(o["flatten_ids"])
        first = int(r_off[ci].reshape(-1)[0])
        end = int(r_off[ci + 1].reshape(-1)[0]) if ci + 1 < C else n_rig
        assert first == total, (ci, first, total)
        assert np.array_equal(r_off[ci] - first, off1), ci
        # the batched ids index the camera-major [C, N] projections: camera ci's are ci * N + Gaussian
        assert np.array_equal(r_fl[first:end].astype(np.int64) - ci * sc.n, fl1), ci
        total += fl1.size
    assert total == n_rig
    print("rig", size, "intersections", n_rig, flush=True)
    want = {k: np_(v).astype(np.float64) for k, v in o["grads"].items() if v is not None}
    assert set(got) == set(want) == {"means", "quats", "log_scales", "opacity_logits", "sh"}
    for k in want:
        _close(f"rig {k}", got[k], want[k])


def test_projection_and_rays_into_preallocated_slices(dev):
    """out= of the UT projection and of camera_rays (extension): one camera's results written into its
    slice of a rig's [C, ...] buffers equal the op's own outputs bit for bit; wrong shapes or dtypes,
    and a pack that needs a gradient, are rejected."""
    sc = S.make_cfg4(seed=5, n=50_000, n_blobs=100)
    st = frame.prepare(sc, dev, requires_grad=False)
    W, H = sc.cameras[0].width, sc.cameras[0].height
    N = sc.means.shape[0]
    scales, opac = torch.exp(st.log_scales), torch.sigmoid(st.opacity_logits)
    C = 2
    fl = torch.full((C, N), 7, dtype=torch.uint8, device=dev)
    ra, m2, de = (torch.full(s, -3.0, device=dev) for s in ((C, N, 2), (C, N, 2), (C, N)))
    ro, rd = torch.full((C, H, W, 3), -3.0, device=dev), torch.full((C, H, W, 3), -3.0, device=dev)
    for c in range(C):
        cam = st.cams[c + 1]
        want = cam.ut_gs_projection(st.means, scales, st.quats, W, H, opacity=opac)
        cam.ut_gs_projection(st.means, scales, st.quats, W, H, opacity=opac, out=(fl[c], ra[c], m2[c], de[c]))
        for a, b in zip((fl[c], ra[c], m2[c], de[c]), want):
            assert torch.equal(a, b)
        wo, wd = cam.camera_rays(W, H)
        go, gd = cam.camera_rays(W, H, out=(ro[c], rd[c]))
        assert go.data_ptr() == ro[c].data_ptr() and gd.data_ptr() == rd[c].data_ptr()
        assert torch.equal(ro[c], wo) and torch.equal(rd[c], wd)
    cam = st.cams[0]
    with pytest.raises(RuntimeError, match="out: flags must be uint8"):
        cam.ut_gs_projection(st.means, scales, st.quats, W, H, opacity=opac, out=(ra[0], ra[0], m2[0], de[0]))
    with pytest.raises(RuntimeError, match="out: tensors for"):
        cam.ut_gs_projection(st.means[:100].contiguous(), scales[:100].contiguous(), st.quats[:100].contiguous(), W,
                             H, opacity=opac[:100].contiguous(), out=(fl[0], ra[0], m2[0], de[0]))
    with pytest.raises(RuntimeError, match="height x width x 3"):
        cam.camera_rays(W, H + 1, out=(ro[0], rd[0]))
    pack = cam.pack.detach().clone().requires_grad_(True)
    with pytest.raises(RuntimeError, match="needs no gradient"):
        cam.ext_cls.camera_rays(pack, W, H, out=(ro[0], rd[0]))


@pytest.mark.parametrize("case", ["static_pinhole", "moving_pinhole", "distorted"])
def test_rig_projection_matches_per_camera(dev, case):
    """projection_utgs_rig (extension: one launch for a rig's cameras of one kind, each Gaussian read
    once) equals projection_utgs per camera bit for bit: the cfg4 rig (static pinholes), the same rig
    with moving poses and moving points, and a distorted-lens rig."""
    sc = S.make_cfg4(seed=7, n=60_000, n_blobs=120)
    specs = sc.cameras
    if case != "static_pinhole":
        specs = [S.CameraSpec(s.kind, s.width, s.height, s.q, s.t, s.impl, v=[1.5, -0.5, 0.1],
                              w=[0.0, 0.02, 0.3], rolling=[0.02, 0.01], trigger_time=0.0, pose_time=0.01)
                 for s in specs]
    if case == "distorted":
        specs = [S.CameraSpec("distorted", s.width, s.height, s.q, s.t, s.impl, v=s.v, w=s.w, rolling=s.rolling,
                              trigger_time=s.trigger_time, pose_time=s.pose_time,
                              dist=[-0.05, 0.01, 0.001, -0.001, 0.0, 0.0, 0.0, 0.0], max_radius=1.5)
                 for s in specs]
    cams = [frame.make_camera(s, dev) for s in specs]
    T = lambda t: t.to(dev).contiguous()
    means, scales, quats, opac = T(sc.means), T(sc.scales), T(sc.quats), T(sc.opacity)
    vel = T(0.5 * torch.randn(sc.means.shape, generator=torch.Generator().manual_seed(3))) \
        if case == "moving_pinhole" else None
    W, H = specs[0].width, specs[0].height
    c0 = cams[0]
    kw = dict(residual_thr_early_stop=c0.residual_thr_early_stop, max_residual=c0.residual_max_valid,
              max_margin=c0.max_margin)
    got = c0.ext_cls.projection_utgs_rig(torch.cat([c.pack for c in cams]), means, vel, scales, quats, opac,
                                         W, H, **kw)
    assert [tuple(x.shape) for x in got] == [(6, 60_000), (6, 60_000, 2), (6, 60_000, 2), (6, 60_000)]
    visible = 0
    for ci, cam in enumerate(cams):
        want = cam.ext_cls.projection_utgs(cam.pack, means, vel, scales, quats, opac, W, H, **kw)
        for name, a, b in zip(("flags", "radii", "means2d", "depths"), got, want):
            assert torch.equal(a[ci], b), (case, ci, name)
        visible += int((want[0] > 0).sum())
    print(case, "visible (camera, Gaussian) pairs", visible, flush=True)
    assert visible > 60_000 // 2
    with pytest.raises(RuntimeError, match="packs must be"):
        c0.ext_cls.projection_utgs_rig(torch.cat([c.pack for c in cams])[:, :5].contiguous(), means, vel, scales,
                                       quats, opac, W, H)


def test_render_rig_mixed_kinds_matches_camera_loop(dev):
    """A rig of two camera kinds (pinholes and distorted-lens cameras of one image size) projects
    camera by camera into its slices instead of in one launch; its images equal render_frame per camera."""
    sc = S.make_cfg4(seed=9, n=60_000, n_blobs=120)
    sc.cameras = [s if i % 2 == 0 else
                  S.CameraSpec("distorted", s.width, s.height, s.q, s.t, s.impl,
                               dist=[-0.04, 0.01, 0.0005, -0.0005, 0.0, 0.0, 0.0, 0.0], max_radius=1.5)
                  for i, s in enumerate(sc.cameras)]
    st = frame.prepare(sc, dev, requires_grad=False)
    assert frame.rig_batchable(st) and len({type(c) for c in st.cams}) == 2
    with torch.no_grad():
        rig = frame.render_rig(st)
        for ci in range(len(sc.cameras)):
            o = frame.render_frame(st, cam_index=ci)
            for k in ("rgb", "depth", "alpha"):
                assert torch.equal(rig[k][ci], o[k]), (ci, k)
            assert torch.equal(rig["radii"][ci], o["radii"]) and torch.equal(rig["depths"][ci], o["depths"])
