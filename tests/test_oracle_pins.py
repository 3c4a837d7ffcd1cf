"""Pins of the CPU oracle (CPU only, no GPU).

The reference ships no tests, golden vectors or fixtures for this path, and it cannot be built or
imported here. Each oracle function is therefore checked against something independent of its own
formula: closed forms, an independent formulation (geometric overlap, library routines), or
finite differences of the float64 build.
"""
import math

import numpy as np
import pytest
import scipy.special as sps
import torch

from oracle import oracle as O
from xsimgs_amd import synthetic as S


def pinhole_spec(width, height, fx, fy, cx, cy, **kw):
    spec = S.pinhole(width, height, fx, fy, cx, cy)
    for k, v in kw.items():
        setattr(spec, k, v)
    return spec


# ------------------------------------------------------------------ UT weights / projection
def test_ut_weights_closed_form():
    w = O.ut_weights(0.1, 2.0, 0.0, prec="f64")
    lam = 0.01 * 3 - 3
    assert np.allclose(w, [lam / (3 + lam), lam / (3 + lam) + (1 - 0.01 + 2), 1 / (2 * (3 + lam)),
                           math.sqrt(3 + lam)], rtol=1e-12)
    assert np.allclose(w, [-99.0, -96.01, 16.666666666666668, 0.17320508075688773], rtol=1e-9)
    # mean weights sum to one, 2D sigma-point covariance weights too
    assert abs(w[0] + 6 * w[2] - 1) < 1e-12


def test_ut_on_axis_closed_form():
    """Axis-aligned Gaussian on the optical axis: the pinhole map is linear on the x / y sigma
    points, so the UT gives cov2d = diag((fx W s_x / z)^2, (fy H s_y / z)^2) and the principal point."""
    W, H, fx, fy = 200, 100, 150.0, 120.0
    spec = pinhole_spec(W, H, fx, fy, W / 2, H / 2)
    z, sx, sy, sz, op = 7.0, 0.3, 0.2, 0.5, 0.8
    means = np.array([[0.0, 0.0, z]])
    flags, radii, m2, dep = O.project_utgs(spec, means, [[sx, sy, sz]], [[1.0, 0, 0, 0]], [op], W, H, prec="f64")
    assert flags[0] == 1 and dep[0] == z
    assert np.allclose(m2[0], [W / 2, H / 2], atol=1e-9)
    ext = min(3.33, math.sqrt(2 * math.log(op * 255)))
    assert np.allclose(radii[0], [ext * fx * sx / z, ext * fy * sy / z], rtol=1e-9)


def test_ut_small_scale_matches_ewa():
    """Off-axis, rotated, tiny Gaussian: the UT covariance converges to J Sigma J^T (EWA)."""
    W, H, fx, fy, cx, cy = 320, 240, 300.0, 280.0, 150.0, 130.0
    spec = pinhole_spec(W, H, fx, fy, cx, cy)
    mu = np.array([0.7, -0.4, 5.0])
    q = np.array([0.9, 0.2, -0.3, 0.25]); q /= np.linalg.norm(q)
    s = np.array([1.0, 0.6, 0.3]) * 2e-4
    op = 0.9
    _, radii, m2, _ = O.project_utgs(spec, mu[None], s[None], q[None], [op], W, H, prec="f64")
    w, x, y, z = q
    R = np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                  [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                  [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])
    Sig = R @ np.diag(s ** 2) @ R.T
    X, Y, Z = mu
    J = np.array([[fx / Z, 0, -fx * X / Z ** 2], [0, fy / Z, -fy * Y / Z ** 2]])
    C = J @ Sig @ J.T
    ext = min(3.33, math.sqrt(2 * math.log(op * 255)))
    assert np.allclose(radii[0], ext * np.sqrt(np.diag(C)), rtol=1e-3)
    assert np.allclose(m2[0], [fx * X / Z + cx, fy * Y / Z + cy], atol=1e-6)


def test_ut_culling_rules():
    spec = pinhole_spec(64, 64, 64.0, 64.0, 32.0, 32.0)
    means = np.array([[0.0, 0, 5], [0, 0, -5], [100.0, 0, 5], [0, 0, 5]])
    s = np.full((4, 3), 0.1)
    q = np.tile([1.0, 0, 0, 0], (4, 1))
    op = np.array([0.5, 0.5, 0.5, 1.0 / 255.0 * 0.99])    # last one below the 1/255 opacity floor
    flags, radii, m2, dep = O.project_utgs(spec, means, s, q, op, 64, 64)
    assert flags.tolist() == [1, 0, 0, 0]
    assert np.all(radii[1:] == 0) and np.all(m2[1:] == 0) and np.all(dep[1:] == 0)


def test_rolling_shutter_residual_invariant():
    """With camera motion and a rolling shutter, a valid projection's time (the op returns it in
    absolute time, projection_kernels.h:301) agrees with the capture time of the normalised pixel
    it lands on (the Newton fixed point of :201-256), within the early-stop threshold."""
    spec = pinhole_spec(200, 100, 180.0, 180.0, 100.0, 50.0, v=[2.0, 0.3, -0.5], w=[0.05, -0.1, 0.2],
                        rolling=[0.0, 0.03], trigger_time=0.0, pose_time=0.015)
    g = np.random.default_rng(0)
    pts = np.stack([g.uniform(-3, 3, 500), g.uniform(-1.5, 1.5, 500), g.uniform(4, 12, 500)], -1)
    uvdt, mask = O.projection(spec, pts, prec="f64")
    assert mask.sum() > 100
    u, v, d, t = uvdt[mask].T
    pix_time = spec.trigger_time + u * spec.rolling[0] + v * spec.rolling[1]
    assert np.abs(t - pix_time).max() < 1e-4
    # and the motion is real: the static projection of the same points lands elsewhere
    static = pinhole_spec(200, 100, 180.0, 180.0, 100.0, 50.0)
    uv0, m0 = O.projection(static, pts, prec="f64")
    assert np.abs(uv0[mask & m0, :2] - uvdt[mask & m0, :2]).max() > 1e-3


def test_spherical_projection_round_trip():
    """A point along the camera ray of pixel (u, v) projects back to (u, v) (spherical convention
    pair: spherical_to_cartesian of the ray and atan2/asin of the projection)."""
    limits = [0.3, 2 * math.pi, -0.4, 0.7]
    spec = S.CameraSpec("spherical", 64, 32, [1.0, 0, 0, 0], [0.0, 0, 0], limits)
    ro, rd = O.camera_rays(spec, 64, 32, prec="f64")
    pts = (rd * 10.0).reshape(-1, 3)
    uvdt, mask = O.projection(spec, pts, prec="f64")
    u_exp = (np.arange(64) + 0.5) / 64
    v_exp = (np.arange(32) + 0.5) / 32
    uu, vv = np.meshgrid(u_exp, v_exp)
    got_u = uvdt[:, 0].reshape(32, 64) % (2 * math.pi / limits[1])
    assert np.allclose(got_u, uu, atol=1e-9)
    assert np.allclose(uvdt[:, 1].reshape(32, 64), vv, atol=1e-9)
    assert np.allclose(uvdt[:, 2], 10.0)


def test_lidar_rays_use_beam_v():
    _, beam_v, limits = S.lidar_beams(16)
    spec = S.CameraSpec("lidar", 32, 16, [1.0, 0, 0, 0], [0.0, 0, 0], limits, beam_v=beam_v)
    _, rd = O.camera_rays(spec, 32, 16, prec="f64")
    elev = np.arcsin(rd[..., 2])
    expected = limits[2] + beam_v.numpy().astype(np.float64) * limits[3]
    assert np.allclose(elev, expected[:, None], atol=1e-6)
    # beams were built top first: +15 deg down to -25 deg at the beam centres
    assert abs(math.degrees(elev[0, 0]) - 15.0) < 1e-3 and abs(math.degrees(elev[-1, 0]) + 25.0) < 1e-3


def test_pinhole_rays_closed_form():
    spec = pinhole_spec(8, 6, 10.0, 12.0, 4.0, 3.0)
    ro, rd = O.camera_rays(spec, 8, 6, prec="f64")
    px, py = np.meshgrid(np.arange(8) + 0.5, np.arange(6) + 0.5)
    d = np.stack([(px - 4.0) / 10.0, (py - 3.0) / 12.0, np.ones_like(px)], -1)
    d /= np.linalg.norm(d, axis=-1, keepdims=True)
    assert np.allclose(rd, d, atol=1e-12) and np.all(ro == 0)


# ------------------------------------------------------------------ spherical harmonics
def _basis(deg, dirs, prec="f64"):
    """oracle basis values via one-hot coefficients"""
    n = dirs.shape[0]
    K = (deg + 1) ** 2
    out = np.zeros((n, K))
    for k in range(K):
        c = np.zeros((n, K, 3))
        c[:, k, 0] = 1.0
        out[:, k] = O.sh_fwd(deg, np.zeros(3), dirs, c, prec=prec)[:, 0] - 0.5
    return out


def _real_sh_scipy(l, m, dirs):
    x, y, z = dirs.T
    polar = np.arccos(np.clip(z, -1, 1))
    az = np.arctan2(y, x)
    Y = sps.sph_harm_y(l, abs(m), polar, az)  # includes the Condon-Shortley phase
    if m > 0:
        return math.sqrt(2) * (-1) ** m * Y.real
    if m < 0:
        return math.sqrt(2) * (-1) ** m * Y.imag
    return Y.real


def test_sh_basis_matches_scipy_real_sh():
    """gsplat's fast SH basis is the real SH with Condon-Shortley phase, bands ordered m = -l..l,
    up to a fixed sign per basis function (pinned here)."""
    g = np.random.default_rng(1)
    d = g.normal(size=(200, 3))
    d /= np.linalg.norm(d, axis=-1, keepdims=True)
    ours = _basis(4, d)
    signs = []
    k = 0
    for l in range(5):
        for m in range(-l, l + 1):
            ref = _real_sh_scipy(l, m, d)
            s = np.sign(np.dot(ours[:, k], ref))
            assert np.allclose(ours[:, k], s * ref, atol=1e-12), (l, m)
            signs.append(int(s))
            k += 1
    assert signs == [(-1) ** k for k in range(25)]   # gsplat flips the sign of every odd basis index


def test_sh_basis_orthonormal():
    """Quadrature over the sphere: int Y_i Y_j = delta_ij (independent of scipy)."""
    nt, nph = 160, 320
    th = (np.arange(nt) + 0.5) * math.pi / nt
    ph = (np.arange(nph) + 0.5) * 2 * math.pi / nph
    T, P = np.meshgrid(th, ph, indexing="ij")
    d = np.stack([np.sin(T) * np.cos(P), np.sin(T) * np.sin(P), np.cos(T)], -1).reshape(-1, 3)
    w = (np.sin(T) * (math.pi / nt) * (2 * math.pi / nph)).reshape(-1)
    B = _basis(4, d)
    G = (B * w[:, None]).T @ B
    assert np.allclose(G, np.eye(25), atol=2e-4)


@pytest.mark.parametrize("layout_3kn,with_dc", [(False, False), (True, False), (False, True), (True, True)])
def test_sh_bwd_finite_differences(layout_3kn, with_dc):
    g = np.random.default_rng(2)
    n, deg = 5, 3
    K = 16 - (1 if with_dc else 0)
    pos = g.normal(size=(n, 3)) * 3
    origin = np.array([0.2, -0.1, 0.3])
    coeffs = g.normal(size=(3, K, n)) if layout_3kn else g.normal(size=(n, K, 3))
    dc = (g.normal(size=(3, n)) if layout_3kn else g.normal(size=(n, 3))) if with_dc else None
    w = g.normal(size=(n, 3))
    L = lambda p, c, o, dcc: float((O.sh_fwd(deg, o, p, c, dc=dcc, layout_3kn=layout_3kn, prec="f64") * w).sum())
    dco, ddc, dpos, dori = O.sh_bwd(deg, origin, pos, coeffs, w, dc=dc, layout_3kn=layout_3kn, prec="f64")
    eps = 1e-6
    for arr, grad, name in ((pos, dpos, "pos"), (coeffs, dco, "coeffs"), (origin, dori, "origin")) + \
            (((dc, ddc, "dc"),) if with_dc else ()):
        num = np.zeros_like(arr)
        it = np.nditer(arr, flags=["multi_index"])
        for _ in it:
            i = it.multi_index
            a0 = arr[i]
            arr[i] = a0 + eps; lp = L(pos, coeffs, origin, dc)
            arr[i] = a0 - eps; lm = L(pos, coeffs, origin, dc)
            arr[i] = a0
            num[i] = (lp - lm) / (2 * eps)
        assert np.allclose(grad, num, rtol=1e-6, atol=1e-8), name


def test_sh_masked_outputs_zero():
    g = np.random.default_rng(3)
    n = 70
    pos, coeffs = g.normal(size=(n, 3)), g.normal(size=(n, 9, 3))
    mask = np.array([0xAAAAAAAA, 0x0, 0xFFFFFFFF], np.uint32)
    out = O.sh_fwd(2, np.zeros(3), pos, coeffs, mask=mask)
    keep = np.array([(mask[i // 32] >> (i % 32)) & 1 for i in range(n)], bool)
    assert np.all(out[~keep] == 0) and np.all(out[keep] != 0)


# ------------------------------------------------------------------ binning, sort, offsets
def _tiles_by_overlap(m, r, ts, n):
    """tiles x with tile interval [x, x+1) meeting the open box ((m-r)/ts, (m+r)/ts), clamped to the grid"""
    lo, hi = (m - r) / ts, (m + r) / ts
    return [x for x in range(n) if lo < x + 1 and x < hi]


def test_isect_regular_against_geometric_overlap():
    g = np.random.default_rng(4)
    W, H, ts = 93, 61, 16
    ntx, nty = (W + ts - 1) // ts, (H + ts - 1) // ts
    n = 300
    m2 = np.stack([g.uniform(-20, W + 20, n), g.uniform(-20, H + 20, n)], -1).astype(np.float32)
    radii = g.uniform(0.1, 40, (n, 2)).astype(np.float32)
    radii[::7] = 0          # culled
    m2[5] = [16.0, 32.0]; radii[5] = [16.0, 16.0]   # exactly on tile borders
    depth = g.uniform(1, 50, n).astype(np.float32)
    depth[10:20] = depth[9]  # ties keep Gaussian order
    tpg, ids, fl = O.isect_regular(m2, radii, depth, W, H, ts, ts, sort=False)
    expect_keys, expect_ids = [], []
    for i in range(n):
        if radii[i, 0] <= 0 or radii[i, 1] <= 0:
            assert tpg[i] == 0
            continue
        xs = _tiles_by_overlap(np.float32(m2[i, 0]), np.float32(radii[i, 0]), np.float32(ts), ntx)
        ys = _tiles_by_overlap(np.float32(m2[i, 1]), np.float32(radii[i, 1]), np.float32(ts), nty)
        assert tpg[i] == len(xs) * len(ys)
        dbits = int(np.float32(depth[i]).view(np.int32))
        for y in ys:
            for x in xs:
                expect_keys.append(((y * ntx + x) << 32) | (dbits & 0xFFFFFFFF))
                expect_ids.append(i)
    assert np.array_equal(ids, np.array(expect_keys, np.int64))
    assert np.array_equal(fl, np.array(expect_ids, np.int32))
    # sorted: numpy stable sort of the reference keys over bits [0, 32 + tile_n_bits)
    _, sids, sfl = O.isect_regular(m2, radii, depth, W, H, ts, ts, sort=True)
    bits = 32 + O.tile_n_bits(ntx * nty)
    order = np.argsort(ids.view(np.uint64) & np.uint64((1 << bits) - 1), kind="stable")
    assert np.array_equal(sids, ids[order]) and np.array_equal(sfl, fl[order])
    # offsets: first sorted index of every tile
    off = O.offset_encode(sids, ntx, nty)
    assert np.array_equal(off.reshape(-1), np.searchsorted(sids >> 32, np.arange(ntx * nty), "left"))


def test_sort_pairs_matches_numpy_stable():
    g = np.random.default_rng(5)
    for bits in (13, 41, 45, 64):
        keys = g.integers(-2**63, 2**63 - 1, 5000, dtype=np.int64)
        keys[:2000] = keys[0]
        vals = np.arange(5000, dtype=np.int32)
        k, v = O.sort_pairs(keys, vals, bits)
        mask = np.uint64((1 << bits) - 1) if bits < 64 else np.uint64(2**64 - 1)
        order = np.argsort(keys.view(np.uint64) & mask, kind="stable")
        assert np.array_equal(k, keys[order]) and np.array_equal(v, vals[order])


def test_offset_encode_empty_and_camera_ids():
    assert np.all(O.offset_encode(np.zeros(0, np.int64), 4, 3) == 0)
    # two cameras: camera id above the tile bits (tiling_common.cu:41-44)
    tnb = O.tile_n_bits(12)
    keys = np.array([((0 << tnb | 3) << 32), ((0 << tnb | 3) << 32), ((1 << tnb | 0) << 32), ((1 << tnb | 11) << 32)],
                    np.int64)
    off = O.offset_encode(keys, 4, 3, n_cams=2).reshape(-1)
    expect = np.searchsorted(np.array([3, 3, 12, 23]), np.arange(24), "left")
    assert np.array_equal(off, expect)


def test_mask_radii():
    radii = np.ones((64, 2), np.float32)
    m = np.zeros(64, bool); m[::3] = True
    out = O.mask_radii(radii, mask=m)
    assert np.all(out[m] == 1) and np.all(out[~m] == 0)
    packed = np.array([0x1, 0x80000000], np.uint32)
    out = O.mask_radii(radii, packed=packed)
    assert np.flatnonzero(out[:, 0]).tolist() == [0, 63]


# ------------------------------------------------------------------ compositing
def _one_tile_scene(means, quats, scales, opac, colors, W=15, H=15, f=15.0):
    spec = pinhole_spec(W, H, f, f, W / 2, H / 2)
    ro, rd = O.camera_rays(spec, W, H, prec="f64")
    n = len(means)
    depth = np.asarray(means, np.float64)[:, 2]
    order = np.argsort(depth, kind="stable").astype(np.int32)
    offsets = np.zeros((1, 1), np.int32)
    return spec, ro, rd, offsets, order


def test_eval3d_single_gaussian_closed_form():
    """Ray through the centre: distance zero, alpha = min(0.999, opacity), hit distance = (mu - o).d."""
    means = np.array([[0.0, 0.0, 5.0]])
    colors = np.array([[0.2, 0.5, 0.9]])
    for op in (0.6, 0.9995):
        spec, ro, rd, off, order = _one_tile_scene(means, None, None, None, None)
        rgb, dep, alp, last = O.eval3d_fwd(means, [[1.0, 0, 0, 0]], [[0.3, 0.2, 0.4]], colors, [op], ro, rd, off,
                                           order, 15, 15, prec="f64")
        a = min(0.999, op)
        assert np.allclose(alp[7, 7], a) and np.allclose(rgb[7, 7], colors[0] * a)
        assert np.allclose(dep[7, 7], a * 5.0)
        assert last[7, 7] == 0


def test_eval3d_two_gaussian_composite():
    means = np.array([[0.0, 0.0, 4.0], [0.0, 0.0, 9.0]])
    colors = np.array([[1.0, 0.0, 0.2], [0.0, 1.0, 0.4]])
    quats = [[1.0, 0, 0, 0], [0.8, 0.6, 0, 0]]
    scales = [[0.2, 0.3, 0.5], [0.5, 0.4, 0.3]]
    op = [0.5, 0.7]
    spec, ro, rd, off, order = _one_tile_scene(means, None, None, None, None)
    rgb, dep, alp, last = O.eval3d_fwd(means, quats, scales, colors, op, ro, rd, off, order, 15, 15, prec="f64")
    a1, a2 = op
    assert np.allclose(rgb[7, 7], colors[0] * a1 + colors[1] * a2 * (1 - a1))
    assert np.allclose(alp[7, 7], 1 - (1 - a1) * (1 - a2))
    assert np.allclose(dep[7, 7], a1 * 4.0 + a2 * (1 - a1) * 9.0)
    assert last[7, 7] == 1


def test_eval3d_termination_is_exclusive():
    """A pixel whose next transmittance would fall to <= 1e-4 stops before that Gaussian."""
    means = np.array([[0.0, 0.0, 3.0 + i] for i in range(6)])
    colors = np.tile([[0.3, 0.3, 0.3]], (6, 1))
    spec, ro, rd, off, order = _one_tile_scene(means, None, None, None, None)
    op = [0.9] * 6
    rgb, dep, alp, last = O.eval3d_fwd(means, [[1.0, 0, 0, 0]] * 6, [[0.5, 0.5, 0.5]] * 6, colors, op, ro, rd, off,
                                       order, 15, 15, prec="f64")
    # T after k Gaussians: 0.1**k; the 4th would give 1e-4 (<= 1e-4): only three are composited
    assert last[7, 7] == 2 and np.allclose(alp[7, 7], 1 - 0.1 ** 3)


def _fd_scene(seed=6, n=6, W=12, H=12, dynamic=False):
    g = np.random.default_rng(seed)
    means = np.stack([g.uniform(-0.4, 0.4, n), g.uniform(-0.4, 0.4, n), g.uniform(4, 6, n)], -1)
    quats = g.normal(size=(n, 4))
    scales = g.uniform(0.25, 0.45, (n, 3))
    opac = g.uniform(0.2, 0.6, n)        # no clamp: opac * vis stays below 0.99
    colors = g.uniform(0, 1, (n, 3))
    spec = pinhole_spec(W, H, 10.0, 10.0, W / 2, H / 2)
    ro, rd = O.camera_rays(spec, W, H, prec="f64")
    order = np.argsort(means[:, 2], kind="stable").astype(np.int32)
    off = np.zeros((1, 1), np.int32)
    vel = g.normal(size=(n, 3)) * 0.3 if dynamic else None
    rtd = g.uniform(-0.2, 0.2, (H, W)) if dynamic else None
    return means, quats, scales, opac, colors, ro, rd, off, order, vel, rtd


@pytest.mark.parametrize("dynamic", [False, True])
def test_eval3d_bwd_finite_differences(dynamic):
    """fp64 oracle backward equals central differences of the fp64 forward away from clamps and
    thresholds (every alpha of the scene stays in (1/255, 0.99), no termination)."""
    means, quats, scales, opac, colors, ro, rd, off, order, vel, rtd = _fd_scene(dynamic=dynamic)
    H, W = ro.shape[:2]
    g = np.random.default_rng(7)
    wr, wd, wa = g.normal(size=(H, W, 3)), g.normal(size=(H, W)), g.normal(size=(H, W))

    def loss(m=means, q=quats, s=scales, o=opac, c=colors, v=vel, t=rtd):
        rgb, dep, alp, _ = O.eval3d_fwd(m, q, s, c, o, ro, rd, off, order, 16, 16, velocity=v, ray_time_delta=t,
                                        prec="f64")
        return float((rgb * wr).sum() + (dep * wd).sum() + (alp * wa).sum())

    rgb, dep, alp, last = O.eval3d_fwd(means, quats, scales, colors, opac, ro, rd, off, order, 16, 16, velocity=vel,
                                       ray_time_delta=rtd, prec="f64")
    gr = O.eval3d_bwd(means, quats, scales, colors, opac, ro, rd, off, order, alp, last, wr, wd, wa, 16, 16,
                      velocity=vel, ray_time_delta=rtd, prec="f64")
    eps = 1e-6
    checks = [("v_means", means, "m"), ("v_quats", quats, "q"), ("v_scales", scales, "s"), ("v_opacity", opac, "o"),
              ("v_colors", colors, "c")]
    if dynamic:
        checks += [("v_velocity", vel, "v"), ("v_time_delta", rtd, "t")]
    for key, arr, kw in checks:
        num = np.zeros_like(arr)
        it = np.nditer(arr, flags=["multi_index"])
        for _ in it:
            i = it.multi_index
            a0 = arr[i]
            arr[i] = a0 + eps; lp = loss(**{kw: arr})
            arr[i] = a0 - eps; lm = loss(**{kw: arr})
            arr[i] = a0
            num[i] = (lp - lm) / (2 * eps)
        assert np.allclose(gr[key], num, rtol=1e-5, atol=1e-7), key


def test_eval3d_bwd_ray_gradients_finite_differences():
    means, quats, scales, opac, colors, ro, rd, off, order, _, _ = _fd_scene(seed=8, W=6, H=6)
    H, W = ro.shape[:2]
    g = np.random.default_rng(9)
    wr, wd, wa = g.normal(size=(H, W, 3)), g.normal(size=(H, W)), g.normal(size=(H, W))
    rgb, dep, alp, last = O.eval3d_fwd(means, quats, scales, colors, opac, ro, rd, off, order, 16, 16, prec="f64")
    gr = O.eval3d_bwd(means, quats, scales, colors, opac, ro, rd, off, order, alp, last, wr, wd, wa, 16, 16,
                      prec="f64")
    eps = 1e-6
    for key, arr in (("v_ray_o", ro), ("v_ray_d", rd)):
        for i in [(0, 0, 0), (3, 2, 1), (5, 5, 2), (2, 4, 0)]:
            a0 = arr[i]
            arr[i] = a0 + eps
            p = O.eval3d_fwd(means, quats, scales, colors, opac, ro, rd, off, order, 16, 16, prec="f64")
            arr[i] = a0 - eps
            m = O.eval3d_fwd(means, quats, scales, colors, opac, ro, rd, off, order, 16, 16, prec="f64")
            arr[i] = a0
            lp = (p[0] * wr).sum() + (p[1] * wd).sum() + (p[2] * wa).sum()
            lm = (m[0] * wr).sum() + (m[1] * wd).sum() + (m[2] * wa).sum()
            assert np.isclose(gr[key][i], (lp - lm) / (2 * eps), rtol=1e-5, atol=1e-8), (key, i)


def _key(tile, depth):
    """(tile << 32) | sign-extended float32 depth bits (tiling_common.cuh:37-45)"""
    return (int(tile) << 32) | int(np.float32(depth).view(np.int32))


def _span_tiles_spherical(mx, my, rx, ry, u_min, u_max, upt, vpt, n_v):
    """regular angular grid: tiles [x, x+1) x [y, y+1) (tile units) meeting the open box, the
    azimuth clipped to [u_min, u_max]"""
    f = np.float32
    lo, hi = max(f(mx - rx), f(u_min)), min(f(mx + rx), f(u_max))
    if hi <= lo:
        return []
    xs = [x for x in range(int(1 / upt) + 2) if x + 1 > lo / f(upt) and x < hi / f(upt)]
    ys = [y for y in range(n_v) if y + 1 > f(my - ry) / f(vpt) and y < f(my + ry) / f(vpt)]
    return [(y, x) for y in ys for x in xs]


def _span_tiles_lidar(mx, my, rx, ry, u_min, u_max, upt, elev):
    """irregular elevation grid: row y covers (elev[y], elev[y+1]] with the first row open below
    and the last open above; a row is hit when it meets [my - ry, my + ry]"""
    f = np.float32
    lo, hi = max(f(mx - rx), f(u_min)), min(f(mx + rx), f(u_max))
    if hi <= lo:
        return []
    xs = [x for x in range(int(1 / upt) + 2) if x + 1 > lo / f(upt) and x < hi / f(upt)]
    n = len(elev)
    vmin, vmax = f(my - ry), f(my + ry)
    ys = []
    for y in range(n):
        a = -np.inf if y == 0 else elev[y]
        b = np.inf if y == n - 1 else elev[y + 1]
        if a < vmax and vmin <= b:
            ys.append(y)
    return [(y, x) for y in ys for x in xs]


@pytest.mark.parametrize("kind", ["lidar", "spherical"])
def test_isect_spherical_family_against_geometric_overlap(kind):
    g = np.random.default_rng(10)
    W, H = 256, 64
    tsx, tsy = 16, 8
    if kind == "lidar":
        _, beam_v, limits = S.lidar_beams(H)
        spec = S.CameraSpec("lidar", W, H, [1.0, 0, 0, 0], [0.0, 0, 0], limits, beam_v=beam_v)
        elev = beam_v.numpy()[::tsy].astype(np.float32)
    else:
        spec = S.CameraSpec("spherical", W, H, [1.0, 0, 0, 0], [0.0, 0, 0], [0.0, 2 * math.pi, -0.5, 1.0])
        elev = None
    spec.rolling = [0.05, 0.0]
    spec.trigger_time, spec.pose_time = 0.0, 0.02          # u_pose = 0.4
    n = 200
    m2 = np.stack([g.uniform(-10, W + 10, n), g.uniform(-10, H + 10, n)], -1).astype(np.float32)
    radii = g.uniform(0.5, 30, (n, 2)).astype(np.float32)
    depth = g.uniform(1, 80, n).astype(np.float32)
    depth[3] = -2.5                                         # negative depth: sign-extended key
    flags = np.ones(n, np.uint8)
    flags[::11] = 0
    radii[5] = 0
    # seam Gaussians (flag 2): 0.3 m Gaussians 20 m away at azimuth u = 0.435, right of u_pose: the
    # positive-time re-projection keeps them there, and their footprint reaches past the first
    # tile column right of the pose column (u >= 0.4375)
    seam = np.arange(7, n, 13)
    flags[seam] = 2
    phi = 0.435 * 2 * math.pi
    pts = np.zeros((n, 3), np.float32)
    pts[:] = [20 * math.sin(phi), 20 * math.cos(phi), 0.5]     # phi = atan2(-x, -y) + pi
    scale = np.full((n, 3), 0.3, np.float32)
    quat = np.tile(np.array([1, 0, 0, 0], np.float32), (n, 1))
    opac = np.full(n, 0.9, np.float32)
    tpg, ids, fl = O.isect_spherical_family(kind, spec, pts, scale, quat, opac, flags, m2, radii, depth, tsx, tsy,
                                           W, H, elev=elev, sort=False)
    upt = np.float32(tsx) / np.float32(W)
    if kind == "lidar":
        n_az, n_v = (W + tsx - 1) // tsx, len(elev)
        span = lambda mx, my, rx, ry, u0, u1: _span_tiles_lidar(mx, my, rx, ry, u0, u1, upt, elev)
    else:
        n_az, n_v = math.ceil(W / tsx), math.ceil(H / tsy)
        vpt = np.float32(tsy) / np.float32(H)
        span = lambda mx, my, rx, ry, u0, u1: _span_tiles_spherical(mx, my, rx, ry, u0, u1, upt, vpt, n_v)
    off = 0
    seen_seam = 0
    for i in range(n):
        if flags[i] == 0 or radii[i, 0] <= 0 or radii[i, 1] <= 0:
            assert tpg[i] == 0
            continue
        mx, my = np.float32(m2[i, 0]) / np.float32(W), np.float32(m2[i, 1]) / np.float32(H)
        rx, ry = np.float32(radii[i, 0]) / np.float32(W), np.float32(radii[i, 1]) / np.float32(H)
        u1 = np.float32(0.4) if flags[i] == 2 else np.float32(1.0)
        first = span(mx, my, rx, ry, np.float32(0.0), u1)
        got = ids[off:off + len(first)].tolist()
        assert got == [_key(y * n_az + x, depth[i]) for y, x in first], i
        assert np.all(fl[off:off + len(first)] == i)
        off += len(first)
        rest = tpg[i] - len(first)
        if flags[i] == 2:
            # second span: right of the pose column, keyed with the re-projected UT depth (~20.006 m)
            seen_seam += rest > 0
            keys = ids[off:off + rest]
            x = (keys >> 32) % n_az
            assert np.all(x >= math.ceil(0.4 / upt))
            d2 = (keys & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
            assert np.allclose(d2, math.sqrt(400 + 0.25), rtol=1e-4)
            off += rest
        else:
            assert rest == 0
    assert off == ids.shape[0] and seen_seam > 0


def test_eval3d_tile_loop_matches_single_tile():
    """Tiled evaluation (every tile's range holding the full depth-sorted list) equals one tile
    covering the whole image: pins the pixel -> tile -> range bookkeeping of the forward."""
    g = np.random.default_rng(11)
    W, H, n = 40, 24, 60
    spec = pinhole_spec(W, H, 30.0, 30.0, W / 2, H / 2)
    ro, rd = O.camera_rays(spec, W, H)
    means = np.stack([g.uniform(-1, 1, n), g.uniform(-0.6, 0.6, n), g.uniform(3, 6, n)], -1)
    quats = g.normal(size=(n, 4))
    scales = g.uniform(0.1, 0.5, (n, 3))
    opac = g.uniform(0.3, 0.95, n)
    colors = g.uniform(0, 1, (n, 5))
    order = np.argsort(means[:, 2], kind="stable").astype(np.int32)
    one = O.eval3d_fwd(means, quats, scales, colors, opac, ro, rd, np.zeros((1, 1), np.int32), order, W, H)
    ntw, nth = (W + 15) // 16, (H + 7) // 8
    offsets = (np.arange(ntw * nth, dtype=np.int32) * n).reshape(nth, ntw)
    tiled = O.eval3d_fwd(means, quats, scales, colors, opac, ro, rd, offsets, np.tile(order, ntw * nth), 16, 8)
    for a, b in zip(one, tiled[:3]):
        assert np.array_equal(a, b)
    # last_ids index the flattened list (tile t's entries start at t * n) and stay 0 for a pixel
    # that nothing reached
    tile_of = (np.arange(H)[:, None] // 8) * ntw + np.arange(W)[None, :] // 16
    hit = one[2] > 0
    assert np.array_equal((tiled[3] - tile_of * n)[hit], one[3][hit])
    assert np.all(tiled[3][~hit] == 0) and np.all(one[3][~hit] == 0)
    assert (one[2] > 0.5).mean() > 0.3 and (one[3] > 0).mean() > 0.3
