"""Compositor parity on scenes built to stress per-wavefront culling.

Every Gaussian is listed in every tile (depth order), so most (wavefront, Gaussian) pairs are far
apart and skipped unevaluated, while the scenes put Gaussians where the skip test is tight: tiny
Gaussians centred on single pixel rays, opacities at 1/255 and one ulp either side, Gaussians far
away, behind the camera, very flat, and tiles whose pixel count is not a multiple of 64. Skipping
must not change any output: renders, last ids and the number of contributing pairs match the
oracle, gradients to the usual tolerance, and the kernel evaluates no more pairs than the oracle.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from xsimgs_amd import _C
from tests._util import GRAD_ATOL, GRAD_RTOL, RENDER_ATOL, frac_close, np_, report

pytestmark = pytest.mark.gpu

W, H = 52, 38


def _scene(seed, tsx, tsy, shared_origin, dynamic, tiny_ray):
    g = np.random.default_rng(seed)
    f = 40.0
    jj, ii = np.meshgrid(np.arange(W) + 0.5, np.arange(H) + 0.5)
    rd = np.stack([(jj - W / 2) / f, (ii - H / 2) / f, np.ones_like(jj)], -1)
    rd /= np.linalg.norm(rd, axis=-1, keepdims=True)
    ro = np.zeros_like(rd)
    if not shared_origin:
        ro += 0.01 * g.standard_normal(ro.shape)
    keep_depth = np.ones((H, W), bool)
    if tiny_ray:  # |rd|^2 below the bundle's range: culling is off for that wavefront
        rd[5, 7] *= 1e-7
        keep_depth[5, 7] = False  # depth scales with 1/|rd|
    n = 260
    z = np.exp(g.uniform(np.log(0.5), np.log(60.0), n))
    xy = g.uniform(-0.8, 0.8, (n, 2)) * z[:, None] * np.array([W / 2 / f, H / 2 / f])
    means = np.concatenate([xy, z[:, None]], 1)
    means[:8, 2] *= -1.0                                  # behind the camera
    means[8:14] *= 200.0                                  # far away
    log_s = g.uniform(np.log(2e-3), np.log(0.25), (n, 3))
    log_s[14:22, 0] -= 5.0                                # very flat
    scales = np.exp(log_s)
    # tiny Gaussians centred on single pixel rays. Their distances are not powers of two: at t = 8 the
    # float32 centre is exactly 8x the float32 direction, gro is then exactly a multiple of grd, and
    # the oracle's cross product (two rounded products) is exactly zero while the kernel's (one fused
    # multiply-add) keeps the rounding of one product -- both within float32 resolution of |gro|, but
    # the f32 oracle would then look exact on a row that float32 does not determine.
    for k, (pi, pj) in enumerate([(3, 4), (17, 30), (30, 50), (37, 0), (20, 26)]):
        t = 5.3 + 3.0 * k
        means[22 + k] = ro[pi, pj] + t * rd[pi, pj] / np.linalg.norm(rd[pi, pj])
        scales[22 + k] = 1e-3
    quats = g.standard_normal((n, 4))
    opac = g.uniform(0.0, 0.7, n)
    th = np.float32(1.0 / 255.0)
    opac[30:33] = [th, np.nextafter(th, np.float32(1)), np.nextafter(th, np.float32(0))]
    opac[33:40] *= 0.02
    colors = g.uniform(0.0, 1.0, (n, 3))
    vel = rtd = None
    if dynamic:
        vel = 0.5 * g.standard_normal((n, 3))
        rtd = g.uniform(-0.05, 0.05, (H, W))
    order = np.argsort(means[:, 2], kind="stable").astype(np.int32)
    ntx, nty = (W + tsx - 1) // tsx, (H + tsy - 1) // tsy
    flat = np.tile(order, ntx * nty).astype(np.int32)
    offsets = (np.arange(ntx * nty, dtype=np.int32) * n).reshape(nty, ntx)
    f32 = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
    return dict(means=f32(means), quats=f32(quats), scales=f32(scales), opac=f32(opac), colors=f32(colors),
                ro=f32(ro), rd=f32(rd), vel=f32(vel), rtd=f32(rtd), offsets=offsets, flat=flat,
                keep_depth=keep_depth)


CASES = [  # tile, shared origin, dynamic, tiny ray
    ((16, 16), True, False, False),
    ((12, 10), False, False, True),
    ((8, 8), True, False, False),
    ((16, 8), False, True, False),
    ((10, 6), True, True, True),
    ((12, 16), True, False, False),   # 192 pixels: four pixels per lane, 48 lanes
    ((10, 15), False, True, False),   # 150 pixels: four pixels per lane, a ragged last lane
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_cull_exact(dev, case):
    (tsx, tsy), shared, dyn, tiny = CASES[case]
    s = _scene(100 + case, tsx, tsy, shared, dyn, tiny)
    print(f"case {case}: tile {tsx}x{tsy} shared={shared} dynamic={dyn} tiny_ray={tiny}", flush=True)
    T = lambda k: torch.from_numpy(s[k]).to(dev)
    counts = torch.zeros(2, dtype=torch.int64, device=dev)
    if dyn:
        out = _C.rasterize_eval3d_dynamic_fwd(T("means"), T("vel"), T("quats"), T("scales"), T("colors").unsqueeze(0),
                                              T("opac").view(1, -1), W, H, tsx, tsy, T("ro"), T("rd"), T("rtd"),
                                              T("offsets"), T("flat"), pair_counts=counts)
    else:
        out = _C.rasterize_eval3d_fwd(T("means"), T("quats"), T("scales"), T("colors").unsqueeze(0),
                                      T("opac").view(1, -1), W, H, tsx, tsy, T("ro"), T("rd"), T("offsets"),
                                      T("flat"), pair_counts=counts)
    rgb, depth, alpha, last = (np_(x) for x in out)
    ref = O.eval3d_fwd(s["means"], s["quats"], s["scales"], s["colors"], s["opac"], s["ro"], s["rd"], s["offsets"],
                       s["flat"], tsx, tsy, velocity=s["vel"], ray_time_delta=s["rtd"], counters=True)
    npix = W * H
    bar = 1.0 - 2.0 / npix  # a termination decided one ulp apart may flip one pixel
    kd = s["keep_depth"]
    for name, a, b in (("rgb", rgb, ref[0]), ("depth", depth[kd], ref[1][kd]), ("alpha", alpha, ref[2])):
        fc = frac_close(a, b, RENDER_ATOL)
        print(report(name, a, b), "frac", fc)
        assert fc >= bar, name
    assert (last == ref[3]).mean() >= bar
    evaluated, contributing = (int(x) for x in counts.cpu())
    print("pairs: evaluated", evaluated, "of", int(ref[4][0]), "| contributing", contributing, int(ref[4][1]))
    assert abs(contributing - int(ref[4][1])) <= 2
    assert evaluated <= int(ref[4][0])

    g = np.random.default_rng(7 + case)
    vr = (g.standard_normal((H, W, 3)) * 1e-3).astype(np.float32)
    vd = (g.standard_normal((H, W)) * 1e-3).astype(np.float32)
    va = (g.standard_normal((H, W)) * 1e-3).astype(np.float32)
    vd[~kd] = 0.0
    Tn = lambda a: torch.from_numpy(a).to(dev)

    def backward(ray_grads):
        if dyn:
            return _C.rasterize_eval3d_dynamic_bwd(T("means"), T("vel"), T("scales"), T("quats"), T("opac"),
                                                   T("colors"), T("ro"), T("rd"), T("rtd"), tsx, tsy, T("offsets"),
                                                   T("flat"), Tn(alpha), Tn(last), Tn(vr), Tn(vd), Tn(va),
                                                   ray_grads=ray_grads)
        return _C.rasterize_eval3d_bwd(T("means"), T("scales"), T("quats"), T("opac"), T("colors"), T("ro"),
                                       T("rd"), tsx, tsy, T("offsets"), T("flat"), Tn(alpha), Tn(last), Tn(vr),
                                       Tn(vd), Tn(va), ray_grads=ray_grads)

    if dyn:
        names = ["v_means", "v_velocity", "v_quats", "v_scales", "v_opacity", "v_colors", "v_ray_o", "v_ray_d",
                 "v_time_delta"]
    else:
        names = ["v_means", "v_quats", "v_scales", "v_opacity", "v_colors", "v_ray_o", "v_ray_d"]
    # with and without per-pixel ray gradients: the kernels differ (pixels per lane, where the
    # mean gradient and the shared-origin terms are summed)
    runs = [(names, backward(True))]
    runs.append(([n for n in names if n not in ("v_ray_o", "v_ray_d")],
                 [x for n, x in zip(names, backward(False)) if n not in ("v_ray_o", "v_ray_d")]))
    # Gradients of the 1 mm Gaussians centred on pixel rays are ill-conditioned in f32 (the oracle's
    # f32 run misses its f64 run there by as much as the kernel does): judge against the f64 oracle,
    # on every Gaussian / pixel that f32 arithmetic determines, and overall no worse than the f32
    # oracle.
    oargs = (s["means"], s["quats"], s["scales"], s["colors"], s["opac"], s["ro"], s["rd"], s["offsets"], s["flat"],
             alpha, last, vr, vd, va, tsx, tsy)
    okw = dict(velocity=s["vel"], ray_time_delta=s["rtd"])
    rg32, rg64 = O.eval3d_bwd(*oargs, **okw), O.eval3d_bwd(*oargs, prec="f64", **okw)
    close = lambda a, b, f=1.0: np.abs(np.asarray(a, np.float64) - b) <= f * (GRAD_ATOL + GRAD_RTOL * np.abs(b))
    for name, a in ((n, x) for nm, gr in runs for n, x in zip(nm, gr)):
        a, b32, b64 = np_(a), rg32[name], rg64[name]
        if name in ("v_ray_o", "v_ray_d"):
            a, b32, b64 = a[kd], b32[kd], b64[kd]
        ok32, okg = close(b32, b64), close(a, b64)
        # a Gaussian (or pixel) is determined in f32 when the f32 oracle lands within a tenth of
        # the tolerance on all its components
        rows = close(b32, b64, 0.1).reshape(ok32.shape[0], -1).all(-1)
        well = float(okg[rows].mean()) if rows.any() else 1.0
        print(report(name, a, b64), f"| vs f64: kernel {okg.mean():.5f} f32 oracle {ok32.mean():.5f} "
              f"kernel where f32 holds {well:.5f}")
        assert well >= 0.999, name
        assert okg.mean() >= ok32.mean() - 0.005, name


@pytest.mark.parametrize("dyn", [False, True])
@pytest.mark.parametrize("cdim", [0, 1, 5, 9, 16, 17])
def test_channel_counts(dev, cdim, dyn):
    """The backward without ray gradients at 16x16 tiles (four pixels per lane; from 17 channels, where
    colours are read from HBM, the ray-gradient kernel) for channel counts that move the gradient
    components across the 16-lane chunks of the wavefront reduction."""
    print(f"cdim {cdim} dynamic={dyn}", flush=True)
    tsx = tsy = 16
    s = _scene(300 + cdim, tsx, tsy, True, dyn, False)
    g = np.random.default_rng(cdim)
    # no colours at all (depth and alpha only) for cdim 0
    s["colors"] = g.uniform(0.0, 1.0, (s["means"].shape[0], cdim)).astype(np.float32) if cdim else None
    T = lambda k: None if s[k] is None else torch.from_numpy(s[k]).to(dev)
    cols = T("colors").unsqueeze(0) if cdim else None
    if dyn:
        out = _C.rasterize_eval3d_dynamic_fwd(T("means"), T("vel"), T("quats"), T("scales"), cols,
                                              T("opac").view(1, -1), W, H, tsx, tsy, T("ro"), T("rd"), T("rtd"),
                                              T("offsets"), T("flat"))
    else:
        out = _C.rasterize_eval3d_fwd(T("means"), T("quats"), T("scales"), cols,
                                      T("opac").view(1, -1), W, H, tsx, tsy, T("ro"), T("rd"), T("offsets"), T("flat"))
    rgb, depth, alpha, last = (np_(x) for x in out)
    okw = dict(velocity=s["vel"], ray_time_delta=s["rtd"])
    ref = O.eval3d_fwd(s["means"], s["quats"], s["scales"], s["colors"], s["opac"], s["ro"], s["rd"], s["offsets"],
                       s["flat"], tsx, tsy, **okw)
    bar = 1.0 - 2.0 / (W * H)
    for name, a, b in (("rgb", rgb, ref[0]), ("alpha", alpha, ref[2])):
        if a is not None and a.size:
            assert frac_close(a, b, RENDER_ATOL) >= bar, name
    vr = (g.standard_normal((H, W, cdim)) * 1e-3).astype(np.float32) if cdim else None
    vd = (g.standard_normal((H, W)) * 1e-3).astype(np.float32)
    va = (g.standard_normal((H, W)) * 1e-3).astype(np.float32)
    Tn = lambda a: None if a is None else torch.from_numpy(a).to(dev)
    if dyn:
        grads = _C.rasterize_eval3d_dynamic_bwd(T("means"), T("vel"), T("scales"), T("quats"), T("opac"), T("colors"),
                                                T("ro"), T("rd"), T("rtd"), tsx, tsy, T("offsets"), T("flat"),
                                                Tn(alpha), Tn(last), Tn(vr), Tn(vd), Tn(va), ray_grads=False)
        names = ["v_means", "v_velocity", "v_quats", "v_scales", "v_opacity", "v_colors", "v_ray_o", "v_ray_d",
                 "v_time_delta"]
    else:
        grads = _C.rasterize_eval3d_bwd(T("means"), T("scales"), T("quats"), T("opac"), T("colors"), T("ro"), T("rd"),
                                        tsx, tsy, T("offsets"), T("flat"), Tn(alpha), Tn(last), Tn(vr), Tn(vd), Tn(va),
                                        ray_grads=False)
        names = ["v_means", "v_quats", "v_scales", "v_opacity", "v_colors", "v_ray_o", "v_ray_d"]
    oargs = (s["means"], s["quats"], s["scales"], s["colors"], s["opac"], s["ro"], s["rd"], s["offsets"], s["flat"],
             alpha, last, vr, vd, va, tsx, tsy)
    rg32, rg64 = O.eval3d_bwd(*oargs, **okw), O.eval3d_bwd(*oargs, prec="f64", **okw)
    close = lambda a, b, f=1.0: np.abs(np.asarray(a, np.float64) - b) <= f * (GRAD_ATOL + GRAD_RTOL * np.abs(b))
    for name, a in zip(names, grads):
        if a is None:  # ray gradients are skipped up to 16 channels; no colour gradient without colours
            assert (cdim <= 16 and name in ("v_ray_o", "v_ray_d")) or (cdim == 0 and name == "v_colors")
            continue
        a, b32, b64 = np_(a), rg32[name], rg64[name]
        ok32, okg = close(b32, b64), close(a, b64)
        rows = close(b32, b64, 0.1).reshape(ok32.shape[0], -1).all(-1)
        well = float(okg[rows].mean()) if rows.any() else 1.0
        print(report(name, a, b64), f"| vs f64: kernel {okg.mean():.5f} f32 oracle {ok32.mean():.5f} "
              f"kernel where f32 holds {well:.5f}")
        assert well >= 0.999, name
        assert okg.mean() >= ok32.mean() - 0.005, name
