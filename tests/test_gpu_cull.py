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
    ((32, 16), False, True, False),   # 512 pixels: 512-thread forward, two backward wavefronts
    ((32, 32), True, False, False),   # 1024 pixels: the largest tile (1024-thread forward)
    ((30, 30), False, False, True),   # 900 pixels: ragged wavefronts in both kernels
    ((20, 40), True, True, False),    # 800 pixels, dynamic
]


def _forward(dev, s, tsx, tsy, dyn, counts=None):
    T = lambda k: None if s[k] is None else torch.from_numpy(s[k]).to(dev)
    cols = None if s["colors"] is None else T("colors").unsqueeze(0)
    kw = {} if counts is None else dict(pair_counts=counts)
    if dyn:
        out = _C.rasterize_eval3d_dynamic_fwd(T("means"), T("vel"), T("quats"), T("scales"), cols,
                                              T("opac").view(1, -1), W, H, tsx, tsy, T("ro"), T("rd"), T("rtd"),
                                              T("offsets"), T("flat"), **kw)
    else:
        out = _C.rasterize_eval3d_fwd(T("means"), T("quats"), T("scales"), cols, T("opac").view(1, -1), W, H,
                                      tsx, tsy, T("ro"), T("rd"), T("offsets"), T("flat"), **kw)
    return [np_(x) for x in out]


def _backward(dev, s, tsx, tsy, dyn, fwd, vr, vd, va, ray_grads, ppl=0):
    """ppl: the backward's pixels per lane for 129..256-pixel tiles without ray gradients (0 chooses by
    grid size: these small images take 2; the full-size frames take 4)."""
    T = lambda k: None if s[k] is None else torch.from_numpy(s[k]).to(dev)
    Tn = lambda a: None if a is None else torch.from_numpy(a).to(dev)
    alpha, last = fwd[2], fwd[3]
    if dyn:
        grads = _C.rasterize_eval3d_dynamic_bwd(T("means"), T("vel"), T("scales"), T("quats"), T("opac"),
                                                T("colors"), T("ro"), T("rd"), T("rtd"), tsx, tsy, T("offsets"),
                                                T("flat"), Tn(alpha), Tn(last), Tn(vr), Tn(vd), Tn(va),
                                                ray_grads=ray_grads, pixels_per_lane=ppl)
        names = ["v_means", "v_velocity", "v_quats", "v_scales", "v_opacity", "v_colors", "v_ray_o", "v_ray_d",
                 "v_time_delta"]
    else:
        grads = _C.rasterize_eval3d_bwd(T("means"), T("scales"), T("quats"), T("opac"), T("colors"), T("ro"),
                                        T("rd"), tsx, tsy, T("offsets"), T("flat"), Tn(alpha), Tn(last), Tn(vr),
                                        Tn(vd), Tn(va), ray_grads=ray_grads, pixels_per_lane=ppl)
        names = ["v_means", "v_quats", "v_scales", "v_opacity", "v_colors", "v_ray_o", "v_ray_d"]
    return dict(zip(names, grads))


def _oracle_grads(s, tsx, tsy, fwd, vr, vd, va):
    """f32 and f64 oracle gradients, plus two f64 runs whose geometric float32 inputs (means,
    velocities, scales, rotations, ray origins, directions and times) are each moved one ulp up or
    down at random -- the spread a float32 computation cannot resolve."""
    def run(sc, prec):
        return O.eval3d_bwd(sc["means"], sc["quats"], sc["scales"], sc["colors"], sc["opac"], sc["ro"], sc["rd"],
                            s["offsets"], s["flat"], fwd[2], fwd[3], vr, vd, va, tsx, tsy, velocity=sc["vel"],
                            ray_time_delta=sc["rtd"], prec=prec)
    g = np.random.default_rng(99)
    moved = []
    for _ in range(2):
        sc = dict(s)
        for k in ("means", "vel", "scales", "quats", "ro", "rd", "rtd"):
            if s[k] is not None:
                up = g.random(s[k].shape) < 0.5
                sc[k] = np.where(up, np.nextafter(s[k], np.float32(np.inf)),
                                 np.nextafter(s[k], np.float32(-np.inf))).astype(np.float32)
        moved.append(run(sc, "f64"))
    return run(s, "f32"), run(s, "f64"), moved


def _check_grads(got, refs, kd, cdim, ray_grads):
    """Judge the kernel against the f64 oracle on every Gaussian (or pixel) that float32 determines,
    and overall no worse than the f32 oracle. Gradients of Gaussians far smaller than the distance
    to the camera (the 1 mm Gaussians centred on pixel rays, thin ones tens of metres out) move by
    more than the tolerance when a mean or a ray direction moves by one float32 ulp, and the f32
    oracle's own rounding misses its f64 run there by as much as the kernel does."""
    rg32, rg64, moved = refs
    close = lambda a, b, f=1.0: np.abs(np.asarray(a, np.float64) - b) <= f * (GRAD_ATOL + GRAD_RTOL * np.abs(b))
    for name, a in got.items():
        if a is None:  # ray gradients are skipped up to 16 channels; no colour gradient without colours
            assert (not ray_grads and cdim <= 16 and name in ("v_ray_o", "v_ray_d")) or \
                (cdim == 0 and name == "v_colors"), name
            continue
        a, b32, b64, bm = np_(a), rg32[name], rg64[name], [m[name] for m in moved]
        if name in ("v_ray_o", "v_ray_d"):
            a, b32, b64, bm = a[kd], b32[kd], b64[kd], [m[kd] for m in bm]
        ok32, okg = close(b32, b64), close(a, b64)
        # determined in f32: the f32 oracle lands within a tenth of the tolerance and the one-ulp
        # moves stay within a quarter of it, on every component of the row
        det = close(b32, b64, 0.1)
        for m in bm:
            det &= close(m, b64, 0.25)
        rows = det.reshape(ok32.shape[0], -1).all(-1)
        well = float(okg.reshape(ok32.shape[0], -1).all(-1)[rows].mean()) if rows.any() else 1.0
        print(report(name, a, b64), f"| vs f64: kernel {okg.mean():.5f} f32 oracle {ok32.mean():.5f} "
              f"| rows determined {int(rows.sum())}/{rows.size}, kernel right on {well:.5f}")
        assert rows.mean() >= 0.9, name
        assert well >= 0.999, name
        assert okg.mean() >= ok32.mean() - 0.005, name


def _grad_inputs(g, cdim):
    vr = (g.standard_normal((H, W, cdim)) * 1e-3).astype(np.float32) if cdim else None
    vd = (g.standard_normal((H, W)) * 1e-3).astype(np.float32)
    va = (g.standard_normal((H, W)) * 1e-3).astype(np.float32)
    return vr, vd, va


@pytest.mark.parametrize("case", range(len(CASES)))
def test_cull_exact(dev, case):
    (tsx, tsy), shared, dyn, tiny = CASES[case]
    s = _scene(100 + case, tsx, tsy, shared, dyn, tiny)
    print(f"case {case}: tile {tsx}x{tsy} shared={shared} dynamic={dyn} tiny_ray={tiny}", flush=True)
    counts = torch.zeros(2, dtype=torch.int64, device=dev)
    fwd = _forward(dev, s, tsx, tsy, dyn, counts)
    rgb, depth, alpha, last = fwd
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

    vr, vd, va = _grad_inputs(np.random.default_rng(7 + case), 3)
    vd[~kd] = 0.0
    refs = _oracle_grads(s, tsx, tsy, fwd, vr, vd, va)
    # with and without per-pixel ray gradients: the kernels differ (pixels per lane, where the
    # mean gradient and the shared-origin terms are summed)
    for ray_grads, ppl in ((True, 0), (False, 4), (False, 2)):
        _check_grads(_backward(dev, s, tsx, tsy, dyn, fwd, vr, vd, va, ray_grads, ppl), refs, kd, 3, ray_grads)


@pytest.mark.parametrize("dyn", [False, True])
@pytest.mark.parametrize("tile", [(16, 16), (12, 16), (10, 15), (16, 8), (32, 16), (32, 32)])
@pytest.mark.parametrize("seed", range(4))
def test_cull_seeds(dev, seed, tile, dyn):
    """The culling scenes over further seeds, at tile shapes with one, four and two pixels per lane,
    a ragged last lane and tiles of 512 and 1024 pixels: renders to the render tolerance, gradients of
    both backward kernels."""
    tsx, tsy = tile
    shared = seed % 2 == 0 and not dyn
    tiny = seed % 3 == 0
    print(f"seed {seed}: tile {tsx}x{tsy} shared={shared} dynamic={dyn} tiny_ray={tiny}", flush=True)
    s = _scene(1000 + seed, tsx, tsy, shared, dyn, tiny)
    fwd = _forward(dev, s, tsx, tsy, dyn)
    ref = O.eval3d_fwd(s["means"], s["quats"], s["scales"], s["colors"], s["opac"], s["ro"], s["rd"], s["offsets"],
                       s["flat"], tsx, tsy, velocity=s["vel"], ray_time_delta=s["rtd"])
    bar = 1.0 - 2.0 / (W * H)
    kd = s["keep_depth"]
    for name, a, b in (("rgb", fwd[0], ref[0]), ("depth", fwd[1][kd], ref[1][kd]), ("alpha", fwd[2], ref[2])):
        assert frac_close(a, b, RENDER_ATOL) >= bar, name
    vr, vd, va = _grad_inputs(np.random.default_rng(seed), 3)
    vd[~kd] = 0.0
    refs = _oracle_grads(s, tsx, tsy, fwd, vr, vd, va)
    for ray_grads, ppl in ((True, 0), (False, 4), (False, 2)):
        _check_grads(_backward(dev, s, tsx, tsy, dyn, fwd, vr, vd, va, ray_grads, ppl), refs, kd, 3, ray_grads)


@pytest.mark.parametrize("dyn", [False, True])
@pytest.mark.parametrize("cdim", [0, 1, 5, 9, 16, 17])
def test_channel_counts(dev, cdim, dyn):
    """The backward without ray gradients at 16x16 tiles (four and two pixels per lane; from 17 channels,
    where colours are read from HBM, the ray-gradient kernel) for channel counts that move the gradient
    components across the 16-lane chunks of the wavefront reduction."""
    print(f"cdim {cdim} dynamic={dyn}", flush=True)
    tsx = tsy = 16
    s = _scene(300 + cdim, tsx, tsy, True, dyn, False)
    g = np.random.default_rng(cdim)
    # no colours at all (depth and alpha only) for cdim 0
    s["colors"] = g.uniform(0.0, 1.0, (s["means"].shape[0], cdim)).astype(np.float32) if cdim else None
    fwd = _forward(dev, s, tsx, tsy, dyn)
    ref = O.eval3d_fwd(s["means"], s["quats"], s["scales"], s["colors"], s["opac"], s["ro"], s["rd"], s["offsets"],
                       s["flat"], tsx, tsy, velocity=s["vel"], ray_time_delta=s["rtd"])
    bar = 1.0 - 2.0 / (W * H)
    for name, a, b in (("rgb", fwd[0], ref[0]), ("alpha", fwd[2], ref[2])):
        if a is not None and a.size:
            assert frac_close(a, b, RENDER_ATOL) >= bar, name
    vr, vd, va = _grad_inputs(g, cdim)
    refs = _oracle_grads(s, tsx, tsy, fwd, vr, vd, va)
    for ppl in (4, 2):
        _check_grads(_backward(dev, s, tsx, tsy, dyn, fwd, vr, vd, va, False, ppl), refs, s["keep_depth"], cdim,
                     False)
