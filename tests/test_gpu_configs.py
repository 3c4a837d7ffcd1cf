"""Parity at the benchmark configurations' full sizes (cfg1 - cfg4 of the benchmark definition).

cfg1 / cfg2: 1M Gaussians, SH3, 1920x1080 pinhole (cfg1 forward, cfg2 forward + backward; cfg2_frustum
the same with every Gaussian inside the field of view: 86M intersections instead of 12M);
cfg3: 3M Gaussians on a ring, 2048x128 spinning-lidar range image with phase modelling, 32x8 tiles,
two colour channels (intensity, ray-drop logit); cfg4: 4M Gaussians in 2000 blobs seen by six
1600x900 pinhole cameras (the reference's equivalent is six single-camera calls, camera.h:58-59;
each camera is one test item here).

Every stage runs on the GPU at full size and is judged against the CPU oracle on the stage's own
GPU inputs (so a stage is judged on its own, with bit-identical inputs on both sides):

* SH colours: within 1e-4 of the oracle on every Gaussian;
* UT projection: flags equal to the f32 oracle's except where float32 does not decide them (a
  decision within a bound on its float32 error, from the f64 oracle's margins), value errors no
  worse than the f32 oracle's (tests/_judge.py);
* binning: tiles per Gaussian, sorted keys, flatten ids and tile offsets (the fill's and
  isect_offset_encode's) bit-exact; for the lidar, a seam Gaussian's second span is a UT
  re-projection inside the binning: its depth bits may differ, and where float32 does not decide
  its tile range (the oracle's seam margins) its tiles too (counted and reported);
* camera rays within 1e-6 / 2e-6;
* composite forward over the whole frame against the f32 oracle: every pixel outside 1e-4 (or
  with another last id) must be one float32 does not determine (an alpha or transmittance
  decision within float32 rounding of its threshold, by the f64 oracle's margins) or right
  against f64;
* composite backward on a fixed subset of tiles (upstream gradients zero elsewhere, the oracle
  run on those tiles): Gaussian gradients judged against f64 as in tests/_judge.py;
* SH backward on the full frame's colour gradients within 1e-3 relative (1e-5 absolute);
* whole-frame properties: finite outputs, alpha in [0, 1], last ids inside their tile's range,
  composited pairs equal to the oracle's up to undetermined pixels, evaluated pairs no more than
  the oracle's, zero gradients for Gaussians no tile lists.
"""
import contextlib

import numpy as np
import pytest
import torch

from oracle import oracle as O
from xsimgs_amd import _C, frame, synthetic
from tests import _judge as J
from tests._util import GRAD_ATOL, GRAD_RTOL, RENDER_ATOL, frac_close, np_, report

pytestmark = pytest.mark.gpu

ITEMS = [("cfg1", 0), ("cfg2", 0), ("cfg2_frustum", 0), ("cfg3", 0)] + [("cfg4", k) for k in range(6)]
_CACHE = {}


class _Stages:
    """Runs every stage's checks and reports all failing stages at the end (the stages' data flow
    does not depend on a check passing)."""

    def __init__(self, label):
        self.label, self.failed = label, []

    @contextlib.contextmanager
    def check(self, name):
        try:
            yield
        except AssertionError as e:
            msg = str(e)[:600]
            self.failed.append(f"{name}: {msg}")
            print(f"{self.label} STAGE FAILED {name}: {msg}", flush=True)


def _scene(name, dev):
    """The configuration's scene on the device (one configuration cached at a time)."""
    if name not in _CACHE:
        _CACHE.clear()
        torch.cuda.empty_cache()
        sc = synthetic.make(name)
        st = frame.prepare(sc, dev, requires_grad=False)
        scales = torch.exp(st.log_scales)
        opac = torch.sigmoid(st.opacity_logits)
        host = dict(means=np_(st.means), quats=np_(st.quats), scales=np_(scales), opac=np_(opac))
        _CACHE[name] = (sc, st, scales, opac, host)
    return _CACHE[name]


def _subset_tiles(n_tiles, k, seed):
    rng = np.random.default_rng(seed)
    t = rng.choice(n_tiles, size=min(k, n_tiles), replace=False)
    return np.unique(np.concatenate([t, [0, n_tiles - 1]])).astype(np.int64)


@pytest.mark.parametrize("name,ci", ITEMS, ids=[f"{n}-cam{c}" for n, c in ITEMS])
def test_config_full_size(dev, name, ci):
    print(f"config {name} camera {ci}", flush=True)
    sc, st, scales, opac, host = _scene(name, dev)
    spec = sc.cameras[ci]
    cam = st.cams[ci]
    W, H = spec.width, spec.height
    tsx, tsy = sc.tile_size
    ntx, nty = (W + tsx - 1) // tsx, (H + tsy - 1) // tsy
    n_tiles = ntx * nty
    label = f"{name}/cam{ci}"
    S = _Stages(label)
    means, quats = st.means, st.quats
    hm, hq, hs, ho = host["means"], host["quats"], host["scales"], host["opac"]

    # ---- colours
    with torch.no_grad():
        if st.sh is not None:
            origin = cam.pose.t
            colors = _C.spherical_harmonics_fused_fwd(sc.sh_degree, origin, means, st.sh, None, False)
            ref_col = O.sh_fwd(sc.sh_degree, np_(origin), hm, np_(st.sh))
            print(f"{label} {report('sh_fwd', np_(colors), ref_col)}", flush=True)
            with S.check("sh_fwd"):
                assert frac_close(np_(colors), ref_col, RENDER_ATOL) == 1.0
        else:
            colors = st.colors
    hc = np_(colors)

    # ---- UT projection
    with torch.no_grad():
        flags, radii, m2, dep = cam.ut_gs_projection(means, scales, quats, W, H, opacity=opac, use_phm=sc.use_phm)
    with S.check("ut_projection"):
        J.judge_ut((flags, radii, m2, dep), spec, hm, hs, hq, ho, W, H, phm=sc.use_phm, label=label)
    hf, hr, hm2, hd = np_(flags), np_(radii), np_(m2), np_(dep)

    # ---- binning on the GPU's projections, tile offsets from the fill and from the encoder
    off_fill = torch.full((nty, ntx), -7, dtype=torch.int32, device=dev)
    with torch.no_grad():
        tpg, ids, fl = cam.isect_gs_tiles(means, scales, quats, W, H, flags, radii, m2, dep, opacity=opac,
                                          tile_size_x=tsx, tile_size_y=tsy, tile_offsets=off_fill)
        off = _C.isect_offset_encode(ids, ntx, nty)
    elev = spec.beam_v.numpy()[::tsy] if spec.kind == "lidar" else None
    ref_in = None
    if spec.kind == "pinhole":
        ref_bin = O.isect_regular(hm2, hr, hd, W, H, tsx, tsy)
    else:
        unsorted = O.isect_spherical_family(spec.kind, spec, hm, hs, hq, ho, hf, hm2, hr, hd, tsx, tsy, W, H,
                                            elev=elev, sort=False)
        ref_bin = (unsorted[0],) + O.sort_pairs(unsorted[1], unsorted[2], 32 + O.tile_n_bits(n_tiles))
        if not any(spec.v) and not any(spec.w):
            # a static camera: both spans of a seam Gaussian carry its input depth in the reference
            ref_in = J.with_input_depths(unsorted, hd, n_tiles)
    hfl, hids = np_(fl), np_(ids)
    und = None
    if spec.kind != "pinhole":
        und = O.isect_spherical_family(spec.kind, spec, hm, hs, hq, ho, hf, hm2, hr, hd, tsx, tsy, W, H, elev=elev,
                                       seam_margins=True) < 1.0
    with S.check("binning"):
        fs = lambda g, t: J.first_span_member(spec.kind, spec, g, t, hm2, hr, W, H, tsx, tsy, elev)
        J.check_binning(spec.kind, (np_(tpg), hids, hfl), ref_bin, hf, hd, n_tiles, label, und, fs,
                        ref_input_depths=ref_in)
    hoff = np_(off)
    with S.check("tile_offsets"):
        # the encoder and the fill's offsets on the GPU's keys; the oracle's where the keys agree
        own = O.offset_encode(hids, ntx, nty)
        assert np.array_equal(hoff, own), f"{label}: isect_offset_encode differs"
        assert np.array_equal(np_(off_fill), own), f"{label}: fill's tile offsets differ"
        if np.array_equal(np_(tpg), ref_bin[0]):
            assert np.array_equal(hoff, O.offset_encode(ref_bin[1], ntx, nty)), label

    # ---- camera rays
    with torch.no_grad():
        ro, rd = cam.camera_rays(W, H)
    rro, rrd = O.camera_rays(spec, W, H)
    hro, hrd = np_(ro), np_(rd)
    with S.check("rays"):
        assert np.abs(hro - rro).max() <= 1e-6 and np.abs(hrd - rrd).max() <= 2e-6, label

    # ---- composite forward, whole frame
    pairs = torch.zeros(2, dtype=torch.int64, device=dev)
    with torch.no_grad():
        rgb, depth, alpha, last = _C.rasterize_eval3d_fwd(means, quats, scales, colors.unsqueeze(0), opac.view(1, -1),
                                                          W, H, tsx, tsy, ro, rd, off, fl, pair_counts=pairs)
    got = [np_(rgb), np_(depth), np_(alpha), np_(last)]
    inp = dict(means=hm, quats=hq, scales=hs, opac=ho, colors=hc, ro=hro, rd=hrd)
    ref32 = O.eval3d_fwd(hm, hq, hs, hc, ho, hro, hrd, hoff, hfl, tsx, tsy, counters=True)
    rj = {"outside_f32": 0}
    with S.check("eval3d_fwd"):
        rj = J.judge_renders(got, ref32, inp, hoff, hfl, tsx, tsy, label=label)
    # whole-frame properties
    starts = hoff.reshape(-1).astype(np.int64)
    ends = np.append(starts[1:], hids.size)
    with S.check("eval3d_fwd_properties"):
        for a in got[:3]:
            assert np.all(np.isfinite(a))
        assert np.all((got[2] >= 0) & (got[2] <= 1))
        tile_of = (np.arange(H)[:, None] // tsy) * ntx + (np.arange(W)[None, :] // tsx)
        lastv = got[3].astype(np.int64)
        contributed = got[2] > 0
        assert np.all(lastv[~contributed] == 0)
        assert np.all((lastv[contributed] >= starts[tile_of][contributed]) & (lastv[contributed] < ends[tile_of][contributed]))
        evaluated, composited = (int(x) for x in pairs.cpu())
        print(f"{label} pairs: kernel evaluated {evaluated} composited {composited} | oracle evaluated {int(ref32[4][0])} "
              f"composited {int(ref32[4][1])}", flush=True)
        assert evaluated <= int(ref32[4][0])
        # a pixel that stops or takes an alpha-threshold Gaussian differently changes the count by a few
        assert abs(composited - int(ref32[4][1])) <= 4 * (rj["outside_f32"] + 1)
    if not sc.backward:
        assert not S.failed, S.failed
        return

    # ---- composite backward: whole frame (the frame's path), then a tile subset against the oracle
    g_rgb, g_dep, g_alp = (g.numpy() for g in (sc.grad_rgb[ci], sc.grad_depth[ci], sc.grad_alpha[ci]))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    with torch.no_grad():
        full = _C.rasterize_eval3d_bwd(means, scales, quats, opac, colors, ro, rd, tsx, tsy, off, fl, alpha, last,
                                       T(g_rgb), T(g_dep), T(g_alp), False)
    names = ["v_means", "v_quats", "v_scales", "v_opacity", "v_colors"]
    listed = np.zeros(hm.shape[0], bool)
    listed[hfl] = True
    with S.check("eval3d_bwd_properties"):
        for nm, a in zip(names, full[:5]):
            a = np_(a)
            assert np.all(np.isfinite(a)), nm
            assert not np.any(a[~listed]), f"{label} {nm}: gradient for a Gaussian no tile lists"
    tiles = _subset_tiles(n_tiles, 192 if n_tiles > 2000 else 96, seed=17 + ci)
    pm = J.tile_pixel_mask(tiles, tsx, tsy, ntx, H, W)
    vr, vd, va = g_rgb * pm[..., None], g_dep * pm, g_alp * pm
    ray_grads = name == "cfg2"   # the per-pixel ray gradients once, on the headline frame
    with torch.no_grad():
        sub = _C.rasterize_eval3d_bwd(means, scales, quats, opac, colors, ro, rd, tsx, tsy, off, fl, alpha, last,
                                      T(vr), T(vd), T(va), ray_grads)
    refs = J.bwd_runs(inp, hoff, hfl, got[2], got[3], vr, vd, va, tsx, tsy, tiles)
    rows = np.unique(np.concatenate([hfl[starts[t]:ends[t]] for t in tiles] + [np.zeros(0, np.int32)]))
    with S.check("eval3d_bwd"):
        J.judge_grads(dict(zip(names, sub[:5])), refs, rows, label=label)
    if ray_grads:
        for nm, a in (("v_ray_o", sub[5]), ("v_ray_d", sub[6])):
            a = np_(a)
            assert not np.any(a[~pm]), nm
            b32, b64 = refs[0][nm][pm], refs[1][nm][pm]
            ok32 = frac_close(b32, b64, GRAD_ATOL, GRAD_RTOL)
            okg = frac_close(a[pm], b64, GRAD_ATOL, GRAD_RTOL)
            print(f"{label} {report(nm, a[pm], b64)} kernel {okg:.5f} f32 oracle {ok32:.5f}", flush=True)
            with S.check("eval3d_bwd_ray_grads"):
                assert okg >= ok32 - 0.005, nm

    # ---- SH backward on the whole frame's colour gradients
    if st.sh is not None:
        v_col = full[4]
        with torch.no_grad():
            dco, _, dpos, dori = _C.spherical_harmonics_fused_bwd(sc.sh_degree, origin, means, st.sh, None, False,
                                                                 v_col, None)
        rdco, _, rdpos, rdori = O.sh_bwd(sc.sh_degree, np_(origin), hm, np_(st.sh), np_(v_col))
        for nm, a, b in (("d_coeffs", dco, rdco), ("d_positions", dpos, rdpos), ("d_origin", dori, rdori)):
            fc = frac_close(np_(a), b, GRAD_ATOL, GRAD_RTOL)
            print(f"{label} {report(nm, np_(a), b)} frac {fc}", flush=True)
            with S.check("sh_bwd"):
                assert fc == 1.0, nm
    assert not S.failed, S.failed
