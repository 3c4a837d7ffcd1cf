"""Judging float32 GPU results against the CPU oracle where float32 rounding decides the outcome.

A value is *determined* in float32 when the float32 oracle lands within a tenth of the tolerance of
the float64 oracle and two float64 runs whose inputs are each moved one float32 ulp at random stay
within a quarter of it: then any faithful float32 implementation must be within the tolerance, and
the kernel is required to be. Elsewhere (a threshold decided by the last bits: alpha at 1/255, the
transmittance cut-off at 1e-4, a UT validity test) the outcome depends on rounding, and such values
are counted and reported rather than required to agree.
"""
import numpy as np

from oracle import oracle as O
from tests._util import GRAD_ATOL, GRAD_RTOL, RENDER_ATOL, np_, report


def move_ulp(a, rng):
    """Every element moved one float32 ulp up or down at random."""
    if a is None:
        return None
    a = np.asarray(a, np.float32)
    up = rng.random(a.shape) < 0.5
    return np.where(up, np.nextafter(a, np.float32(np.inf)), np.nextafter(a, np.float32(-np.inf))).astype(np.float32)


def tiles_of_pixels(pix_rows, pix_cols, tsx, tsy, ntx):
    return np.unique((pix_rows // tsy) * ntx + (pix_cols // tsx))


def tile_pixel_mask(tiles, tsx, tsy, ntx, H, W):
    m = np.zeros((H, W), bool)
    for t in np.asarray(tiles):
        ty, tx = divmod(int(t), ntx)
        m[ty * tsy:(ty + 1) * tsy, tx * tsx:(tx + 1) * tsx] = True
    return m


# ------------------------------------------------------------------ forward renders
def fwd_runs(inp, off, fl, tsx, tsy, tiles, seed=0):
    """f32 and f64 oracle renders on `tiles`, plus two f64 runs with one-ulp moved inputs."""
    rng = np.random.default_rng(seed)

    def run(d, prec, margins=False):
        return O.eval3d_fwd(d["means"], d["quats"], d["scales"], d["colors"], d["opac"], d["ro"], d["rd"], off, fl,
                            tsx, tsy, velocity=d.get("vel"), ray_time_delta=d.get("rtd"), prec=prec, tiles=tiles,
                            margins=margins)
    moved = []
    for _ in range(2):
        d = dict(inp)
        for k in ("means", "quats", "scales", "opac", "ro", "rd", "vel", "rtd"):
            if d.get(k) is not None:
                d[k] = move_ulp(d[k], rng)
        moved.append(run(d, "f64"))
    return run(inp, "f32"), run(inp, "f64", margins=True), moved


def judge_renders(got, ref32_full, inp, off, fl, tsx, tsy, keep_depth=None, label=""):
    """Full-frame renders (rgb or None, depth, alpha, last_ids) against the f32 oracle's; every pixel
    outside RENDER_ATOL (or with another last id) is classified with f64 runs on its tile: undetermined
    when one of the pixel's threshold decisions (alpha at 1/255, the transmittance cut-off) lies within
    a bound on float32 rounding (the f64 oracle's margins), or the f32 oracle or a one-ulp moved f64
    run leaves the tolerance. Asserts that each such pixel is undetermined or right against f64."""
    rgb, depth, alpha, last = got
    r_rgb, r_dep, r_alp, r_last = ref32_full[:4]
    H, W = alpha.shape
    ntx = off.shape[-1]
    kd = np.ones((H, W), bool) if keep_depth is None else keep_depth

    def bad_of(a_rgb, a_dep, a_alp, b_rgb, b_dep, b_alp, f=1.0):
        t = f * RENDER_ATOL
        bad = np.abs(np.asarray(a_alp, np.float64) - b_alp) > t
        bad |= kd & (np.abs(np.asarray(a_dep, np.float64) - b_dep) > t)
        if a_rgb is not None and a_rgb.size:
            bad |= (np.abs(np.asarray(a_rgb, np.float64) - b_rgb) > t).any(-1)
        return bad
    bad = bad_of(rgb, depth, alpha, r_rgb, r_dep, r_alp) | (last != r_last)
    n_bad = int(bad.sum())
    out = dict(pixels=H * W, outside_f32=n_bad, undetermined=0, right_vs_f64=0)
    for name, a, b in (("rgb", rgb, r_rgb), ("depth", depth[kd], r_dep[kd]), ("alpha", alpha, r_alp)):
        if a is not None and a.size:
            print(f"{label} {report(name, a, b)}", flush=True)
    if n_bad:
        ii, jj = np.nonzero(bad)
        tiles = tiles_of_pixels(ii, jj, tsx, tsy, ntx)
        r32, r64, moved = fwd_runs(inp, off, fl, tsx, tsy, tiles)
        undet = bad_of(r32[0], r32[1], r32[2], r64[0], r64[1], r64[2], 0.1) | (r32[3] != r64[3])
        undet |= r64[4] < 1.0   # a threshold decision within float32 rounding (oracle margins)
        for m in moved:
            undet |= bad_of(m[0], m[1], m[2], r64[0], r64[1], r64[2], 0.25) | (m[3] != r64[3])
        right = ~bad_of(rgb, depth, alpha, r64[0], r64[1], r64[2]) & (last == r64[3])
        undet_b, right_b = undet[bad], right[bad]
        out["undetermined"] = int(undet_b.sum())
        out["right_vs_f64"] = int((right_b & ~undet_b).sum())
        wrong = bad & ~undet & ~right
        if wrong.any():
            wi, wj = np.nonzero(wrong)
            for i, j in list(zip(wi, wj))[:5]:
                print(f"{label} WRONG pixel ({i},{j}): gpu a={alpha[i, j]:.7g} d={depth[i, j]:.7g} last={last[i, j]} | "
                      f"f32 a={r_alp[i, j]:.7g} d={r_dep[i, j]:.7g} last={r_last[i, j]} | f64 a={r64[2][i, j]:.7g} "
                      f"d={r64[1][i, j]:.7g} last={r64[3][i, j]}", flush=True)
        out["wrong"] = int(wrong.sum())
    else:
        out["wrong"] = 0
    print(f"{label} renders: {out}", flush=True)
    assert out["wrong"] == 0, out
    return out


# ------------------------------------------------------------------ gradients
def bwd_runs(inp, off, fl, alpha, last, vr, vd, va, tsx, tsy, tiles, seed=99):
    rng = np.random.default_rng(seed)

    def run(d, prec, abs_sums=False, und_mode=0):
        return O.eval3d_bwd(d["means"], d["quats"], d["scales"], d["colors"], d["opac"], d["ro"], d["rd"], off, fl,
                            alpha, last, vr, vd, va, tsx, tsy, velocity=d.get("vel"), ray_time_delta=d.get("rtd"),
                            prec=prec, tiles=tiles, abs_sums=abs_sums, und_mode=und_mode)
    moved = []
    for _ in range(2):
        d = dict(inp)
        for k in ("means", "quats", "scales", "ro", "rd", "vel", "rtd"):
            if d.get(k) is not None:
                d[k] = move_ulp(d[k], rng)
        moved.append(run(d, "f64"))
    # every pair whose alpha test or geometry gate float32 rounding can decide either way taken, and dropped
    forced = [run(inp, "f64", und_mode=1), run(inp, "f64", und_mode=2)]
    return run(inp, "f32"), run(inp, "f64", abs_sums=True), moved, forced


# A float32 sum of per-pair contributions t_i, in any order, each term carrying its own rounding, is off
# by at most about C_SUM * u * sum |t_i| (u = 2^-24; C_SUM covers the per-pair chain's roundings, the
# 64-lane reduction and the atomics across wavefronts). Where that is not below a quarter of the
# tolerance, the summation order alone can decide the comparison.
F32_U = 2.0 ** -24
C_SUM = 64.0


def judge_grads(got, refs, rows, label="", min_determined=0.85):
    """Per-Gaussian (or per-pixel) gradients on `rows` (the Gaussians the judged pixels reach); every
    other row must be exactly zero. An element is determined in float32 when the f32 oracle lies within
    a tenth of the tolerance of f64, two f64 runs with one-ulp moved inputs within a quarter, the
    float32 summation bound of its contributions (C_SUM u sum|t_i|, from the f64 oracle) within a
    quarter, and the f64 runs that take and that drop every pair whose alpha test or geometry gate
    float32 rounding decides (refs[3], when given) within a quarter; a row is determined when all its
    elements are. Every determined row must be right (any miss fails, with its values printed), at
    least `min_determined` of the rows must be determined, and overall the kernel may be no worse
    against f64 than the f32 oracle. Returns per-name stats."""
    rg32, rg64, moved = refs[:3]
    forced = refs[3] if len(refs) > 3 else []
    tol = lambda b: GRAD_ATOL + GRAD_RTOL * np.abs(b)
    close = lambda a, b, f=1.0: np.abs(np.asarray(a, np.float64) - b) <= f * tol(b)
    absd = rg64.get("abs", {})
    stats = {}
    for name, a in got.items():
        if a is None or name not in rg64 or rg64[name] is None:
            continue
        a = np_(a)
        other = np.ones(a.shape[0], bool)
        other[rows] = False
        assert not np.any(a[other]), f"{label} {name}: gradient outside the judged Gaussians"
        a, b32, b64, bm = a[rows], rg32[name][rows], rg64[name][rows], [m[name][rows] for m in moved]
        ok32, okg = close(b32, b64), close(a, b64)
        det = close(b32, b64, 0.1)
        for m in bm:
            det &= close(m, b64, 0.25)
        thr_ok = np.ones_like(det)
        for fr in forced:
            thr_ok &= close(fr[name][rows], b64, 0.25)
        det &= thr_ok
        cond_ok = np.ones_like(det)
        if absd.get(name) is not None:
            cond_ok = C_SUM * F32_U * absd[name][rows] <= 0.25 * tol(b64)
            det &= cond_ok
        nr = a.shape[0]
        drow = det.reshape(nr, -1).all(-1)
        right = okg.reshape(nr, -1).all(-1)
        miss = np.nonzero(drow & ~right)[0]
        well = float(right[drow].mean()) if drow.any() else 1.0
        stats[name] = dict(rows=nr, determined=round(float(drow.mean()), 5),
                           cancelling=round(float(1.0 - cond_ok.reshape(nr, -1).all(-1).mean()), 5),
                           threshold_decided=round(float(1.0 - thr_ok.reshape(nr, -1).all(-1).mean()), 5),
                           kernel_right_on_determined=round(well, 6), kernel_vs_f64=round(float(okg.mean()), 6),
                           f32_oracle_vs_f64=round(float(ok32.mean()), 6))
        print(f"{label} {report(name, a, b64)} | {stats[name]}", flush=True)
        for r in miss[:10]:
            ab = absd[name][rows][r] if absd.get(name) is not None else None
            print(f"{label} {name} MISS row {rows[r]}: kernel {np.ravel(a[r])} f32 {np.ravel(b32[r])} "
                  f"f64 {np.ravel(b64[r])} moved {[np.ravel(m[r]) for m in bm]} sum|t| {np.ravel(ab)}", flush=True)
        assert drow.mean() >= min_determined, (name, stats[name])
        assert miss.size == 0, (name, stats[name], [int(rows[r]) for r in miss[:10]])
        assert okg.mean() >= ok32.mean() - 0.005, (name, stats[name])
    return stats


def judge_pixel_grads(got, refs, pixel_mask, label="", min_determined=0.85):
    """Per-pixel gradients (v_ray_o, v_ray_d, v_time_delta: [H, W(, k)]) judged as judge_grads judges
    per-Gaussian rows, one row per pixel of `pixel_mask` (pixels outside it must be exactly zero)."""
    rg32, rg64, moved = refs[:3]
    forced = refs[3] if len(refs) > 3 else []
    hw = pixel_mask.size
    flat = lambda d: {k: (None if d.get(k) is None else np.asarray(d[k]).reshape(hw, -1)) for k in got}
    r64 = flat(rg64)
    r64["abs"] = flat(rg64.get("abs", {}))
    g = {k: np_(v).reshape(hw, -1) for k, v in got.items()}
    return judge_grads(g, (flat(rg32), r64, [flat(m) for m in moved], [flat(f) for f in forced]),
                       np.nonzero(pixel_mask.reshape(-1))[0], label=label, min_determined=min_determined)


# ------------------------------------------------------------------ binning
def first_span_member(kind, spec, gids, tiles, means2d, radii, W, H, tsx, tsy, elev=None):
    """For entries (Gaussian, tile) of seam Gaussians: True where the tile lies in the Gaussian's first
    span, the one binned from its input projection on one side of u_pose (phm_lidar_tiling.cu:146-175,
    tile_limits_irregular :52-91; phm_spherical_tiling.cu tile_limits_regular :15-45), recomputed
    here in float32 with the reference's operations."""
    f = np.float32
    roll = f(spec.rolling[0])
    u_pose = f((f(spec.pose_time) - f(spec.trigger_time)) / roll) if abs(roll) > 0 else f(0.5)
    m = means2d[gids].astype(f)
    r = radii[gids].astype(f)
    mx, my = m[:, 0] / f(W), m[:, 1] / f(H)
    rx, ry = r[:, 0] / f(W), r[:, 1] / f(H)
    u_min = np.full(gids.shape, f(0.0), f)
    u_max = np.full(gids.shape, f(1.0), f)
    if roll > 0:
        u_max[:] = u_pose
    else:
        u_min[:] = u_pose
    lo, hi = np.maximum(mx - rx, u_min), np.minimum(mx + rx, u_max)
    ut = f(tsx) / f(W)
    x0 = np.floor(lo / ut).astype(np.int64)
    if kind == "lidar":
        x1 = np.ceil(hi / ut).astype(np.int64) - 1
        n_az = (int(W) + tsx - 1) // tsx
        e = np.asarray(elev, f)
        # find_bounds_increasing: index of the last boundary below the value, clamped to [0, n - 1]
        y0 = np.clip(np.searchsorted(e, my - ry, side="left") - 1, 0, e.size - 1)
        y1 = np.clip(np.searchsorted(e, my + ry, side="left") - 1, 0, e.size - 1)
        y1 = np.maximum(y1, y0)
        ty, tx = tiles // n_az, tiles % n_az
        inside = (tx >= x0) & (tx <= x1) & (ty >= y0) & (ty <= y1)
    else:
        x1 = np.ceil(hi / ut).astype(np.int64)
        n_az = int(np.ceil(f(W) / f(tsx)))
        n_v = int(np.ceil(f(H) / f(tsy)))
        vt = f(tsy) / f(H)
        y0 = np.clip(np.floor((my - ry) / vt).astype(np.int64), 0, n_v)
        y1 = np.clip(np.ceil((my + ry) / vt).astype(np.int64), 0, n_v)
        ty, tx = tiles // n_az, tiles % n_az
        inside = (tx >= x0) & (tx < x1) & (ty >= y0) & (ty < y1)
    return inside & (hi > lo)


def with_input_depths(unsorted, depths, n_tiles):
    """An unsorted binning (tiles per Gaussian, keys, flatten ids) with every key's depth bits replaced by
    its Gaussian's input depth, sorted stably over the reference's key bits: what the reference's
    binning gives a static camera's seam Gaussians, whose re-projected depth (the centre point's range,
    which no phase mode changes) is the stored one (phm_lidar_tiling.cu:199-205 against
    ut_phm_kernels.h:60-95)."""
    tpg, ids, fl = unsorted
    # a key is (tile << 32) + the sign-extended depth bits (tiling_common.cuh:37)
    tile = (ids >> 32) + ((ids & 0xFFFFFFFF) >= (1 << 31))
    d = np.asarray(depths, np.float32).view(np.int32)[fl].astype(np.int64)
    sk, sv = O.sort_pairs((tile << 32) + d, fl.copy(), 32 + O.tile_n_bits(n_tiles))
    return tpg, sk, sv


def check_binning(kind, got, ref, flags, depths, n_tiles, label, undetermined=None, first_span=None,
                  ref_input_depths=None):
    """Bit-exact binning. For the lidar / spherical kinds a seam (flag-2) Gaussian's second span is
    re-projected inside the binning (PositiveDelta UT, phm_lidar_tiling.cu:183-229), so that span's
    depth bits may differ, and where float32 does not decide its tile range (`undetermined`, from the
    oracle's seam margins) its tiles may differ too; every other entry must be identical.

    With `ref_input_depths` (a static camera: the oracle's binning keyed with the input depths, see
    with_input_depths) every key must carry its Gaussian's input depth bits, as in the reference, and
    the sorted keys and flatten ids must equal that oracle's bit for bit outside the undetermined
    seam spans."""
    tpg, ids, fl = got
    rtpg, rids, rfl = ref
    und = np.zeros(tpg.shape[0], bool) if undetermined is None else undetermined
    cnt_diff = np.nonzero(tpg != rtpg)[0]
    assert np.all(und[cnt_diff]), f"{label}: tiles per Gaussian differ at {cnt_diff[~und[cnt_diff]][:10]}"
    if ref_input_depths is not None:
        gbits = (ids & 0xFFFFFFFF).astype(np.uint32)
        want = np.asarray(depths, np.float32).view(np.uint32)[fl]
        bad = np.nonzero(gbits != want)[0]
        assert bad.size == 0, (f"{label}: {bad.size} keys do not carry their Gaussian's input depth "
                               f"(first at entry {bad[:5]}, Gaussians {fl[bad[:5]]}, flags {flags[fl[bad[:5]]]})")
        _, sids, sfl = ref_input_depths
        kg, kr = ~und[fl], ~und[sfl]
        assert np.array_equal(ids[kg], sids[kr]) and np.array_equal(fl[kg], sfl[kr]), \
            f"{label}: keys / flatten ids differ from the oracle's keyed with the input depths"
        print(f"{label}: every key carries its Gaussian's input depth; keys and ids bit-exact against the "
              f"oracle's keyed with the input depths outside {int(und.sum())} undetermined seam spans "
              f"({int(kg.sum())} of {ids.size} entries)", flush=True)
    if kind == "pinhole" or (np.array_equal(ids, rids) and np.array_equal(fl, rfl)):
        assert np.array_equal(ids, rids) and np.array_equal(fl, rfl), label
        print(f"{label}: binning bit-exact, {ids.size} intersections", flush=True)
        return 0
    # drop the undetermined seam Gaussians' entries on both sides; match the rest by (Gaussian, tile)
    keep_g, keep_r = ~und[fl], ~und[rfl]
    tile = lambda k: (k >> 32).astype(np.int64)
    gi, gk = fl[keep_g], ids[keep_g]
    ri, rk = rfl[keep_r], rids[keep_r]
    assert gi.shape == ri.shape, f"{label}: {gi.size} vs {ri.size} entries outside the undetermined spans"
    og = np.lexsort((tile(gk), gi))
    orf = np.lexsort((tile(rk), ri))
    assert np.array_equal(gi[og], ri[orf]) and np.array_equal(tile(gk)[og], tile(rk)[orf]), \
        f"{label}: different (Gaussian, tile) entries"
    k_g, k_r = gk[og], rk[orf]
    diff = k_g != k_r
    g_d = gi[og][diff]
    gbits = (k_g[diff] & 0xFFFFFFFF).astype(np.uint32)
    rbits = (k_r[diff] & 0xFFFFFFFF).astype(np.uint32)
    # only second spans of flag-2 Gaussians (the first span is keyed with the input depth)
    assert np.all(flags[g_d] == 2), f"{label}: a key of a non-seam Gaussian differs"
    if first_span is not None:
        assert not np.any(first_span(g_d, tile(k_g[diff]))), f"{label}: a first-span key differs"
    gv, rv = gbits.view(np.float32).astype(np.float64), rbits.view(np.float32).astype(np.float64)
    assert np.all(np.abs(gv - rv) <= 1e-5 * np.abs(rv)), f"{label}: re-projected depth off by more than 1e-5"
    # sorted, stably, by its own keys over the reference's bits
    bits = 32 + int(np.floor(np.log2(np.float32(n_tiles)))) + 1
    masked = ids.view(np.uint64) & np.uint64((1 << bits) - 1)
    assert np.all(masked[1:] >= masked[:-1])
    tie = masked[1:] == masked[:-1]
    assert np.all(fl[1:][tie] >= fl[:-1][tie])
    # per-tile counts outside the undetermined spans
    assert np.array_equal(np.bincount(tile(gk), minlength=n_tiles), np.bincount(tile(rk), minlength=n_tiles))
    ulps = np.abs(gbits.astype(np.int64) - rbits.astype(np.int64))
    n_diff = int(diff.sum())
    print(f"{label}: {int(und.sum())} seam spans undetermined in float32 ({cnt_diff.size} with another tile count); "
          f"outside them {n_diff} of {gk.size} keys differ, all in re-projected second-span depth bits "
          f"(max {int(ulps.max()) if n_diff else 0} ulp)", flush=True)
    return n_diff


# ------------------------------------------------------------------ UT projection
def judge_ut(got, spec, means, scales, quats, opac, W, H, phm=False, sample=20000, label="", seed=5, vel=None):
    """UT outputs (flags, radii, means2d, depths) against the oracle, on bit-identical inputs.

    Flags: equal to the f32 oracle's except where float32 does not decide them: the f64 oracle's
    margin (a validity decision -- on-screen extent, covariance determinant and signs, the seam's
    u_distance, the projection's bounds -- lies within a bound on its float32 error) is below 1, or
    the f32 oracle itself disagrees with f64. The UT's weighted sums cancel terms about 200 times
    larger than the result (weights -99 and 6 x 16.7 at the defaults, ut_kernels.h:17-36), so
    float32 means2d and radii carry errors of ~1e-2 px at 1000 px. Values, on a sample valid on both
    sides: the distribution of |gpu - f64| may be no worse than twice the f32 oracle's at the
    median, 90th, 99th, 99.9th percentile and maximum. Culled Gaussians' outputs are zero
    (ut_kernels.h:276-280)."""
    gf, gr, gm, gd = (np_(x) for x in got)
    rf, rr, rm, rd = O.project_utgs(spec, means, scales, quats, opac, W, H, vel=vel, phm=phm)
    f64 = O.project_utgs(spec, means, scales, quats, opac, W, H, vel=vel, phm=phm, prec="f64", margins=True)
    rng = np.random.default_rng(seed)
    dis = np.nonzero(gf != rf)[0]
    both = np.nonzero((gf > 0) & (rf > 0))[0]
    samp = np.sort(rng.choice(both, size=min(sample, both.size), replace=False)) if both.size else both
    und_all = (f64[4] < 1.0) | (rf != f64[0])
    undet = und_all[dis]
    wrong = ~undet & (gf[dis] != f64[0][dis])
    out = dict(n=int(gf.size), visible_gpu=int((gf > 0).sum()), flag2=int((gf == 2).sum()),
               flag_disagree=int(dis.size), flag_undetermined=int(undet.sum()), flag_wrong=int(wrong.sum()),
               f32_oracle_vs_f64=int((rf != f64[0]).sum()), undetermined_overall=int(und_all.sum()))
    if wrong.any():
        out["wrong_ids"] = dis[wrong][:8].tolist()
        out["wrong_gpu_oracle"] = [(int(gf[g]), int(rf[g])) for g in dis[wrong][:8]]
        out["wrong_margins"] = [float(f"{f64[4][g]:.3g}") for g in dis[wrong][:8]]
    r64 = [x[samp] for x in f64[:4]]
    vals = {}
    qs = (0.5, 0.9, 0.99, 0.999, 1.0)
    for name, g, r32, j in (("radii", gr, rr, 1), ("means2d", gm, rm, 2), ("depth", gd, rd, 3)):
        ok_rows = (r64[0] > 0) & (gf[samp] == r64[0])
        b64 = np.asarray(r64[j][ok_rows], np.float64)
        eg = np.abs(np.asarray(g[samp][ok_rows], np.float64) - b64).reshape(-1)
        eo = np.abs(np.asarray(r32[samp][ok_rows], np.float64) - b64).reshape(-1)
        floor = 1e-6 * (1.0 + float(np.median(np.abs(b64)))) if b64.size else 0.0
        qg = np.quantile(eg, qs) if eg.size else np.zeros(len(qs))
        qo = np.quantile(eo, qs) if eo.size else np.zeros(len(qs))
        vals[name] = dict(gpu=[float(f"{x:.3g}") for x in qg], f32_oracle=[float(f"{x:.3g}") for x in qo],
                          worse=[q for q, a, b in zip(qs, qg, qo) if a > 2.0 * b + floor])
    out["values_err_quantiles"] = vals
    print(f"{label} UT: {out}", flush=True)
    assert out["flag_wrong"] == 0, out
    for name, v in vals.items():
        assert not v["worse"], (name, v)
    z = gf == 0
    assert not gr[z].any() and not gm[z].any() and not gd[z].any()
    return out
