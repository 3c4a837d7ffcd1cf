"""Writes the golden fixtures beside this file from the CPU oracle (float32 build).

The reference ships no vectors, known-answer tests or fixtures for the rasterization path, and it
cannot be built or imported here, so these fixtures are the oracle's own outputs on small seeded
scenes, every stage fed with the oracle's upstream results. The oracle itself is pinned by
tests/test_oracle_pins.py; the fixtures freeze its outputs so that the GPU path is checked
against committed data and any later change of the oracle shows up as a diff.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from xsimgs_amd import synthetic as S  # noqa: E402

KINDS = {"pinhole": 0, "spherical": 1, "lidar": 2}


def spec_arrays(spec):
    d = dict(cam_kind=np.int32(KINDS[spec.kind]), cam_size=np.array([spec.width, spec.height], np.int32),
             cam_q=np.array(spec.q, np.float32), cam_t=np.array(spec.t, np.float32),
             cam_v=np.array(spec.v, np.float32), cam_w=np.array(spec.w, np.float32),
             cam_rolling=np.array(spec.rolling, np.float32),
             cam_times=np.array([spec.trigger_time, spec.pose_time], np.float32),
             cam_impl=np.array(spec.impl, np.float32))
    if spec.beam_v is not None:
        d["cam_beam_v"] = np.asarray(spec.beam_v, np.float32)
    return d


def _unit_quats(g, n):
    q = g.normal(size=(n, 4))
    return (q / np.linalg.norm(q, axis=-1, keepdims=True)).astype(np.float32)


def _sigmoid(x):
    return (1.0 / (1.0 + np.exp(-x))).astype(np.float32)


def _pixel_time_delta(spec, W, H):
    u = (np.arange(W, dtype=np.float64) + 0.5) / W
    v = (np.arange(H, dtype=np.float64) + 0.5) / H
    t = spec.trigger_time + u[None, :] * spec.rolling[0] + v[:, None] * spec.rolling[1] - spec.pose_time
    return t.astype(np.float32)


def composite(case, spec, W, H, tsx, tsy, means, quats, scales, opac, colors, off, fl, g, vel=None, rtd=None):
    ro, rd = O.camera_rays(spec, W, H)
    rgb, dep, alp, last = O.eval3d_fwd(means, quats, scales, colors, opac, ro, rd, off, fl, tsx, tsy,
                                       velocity=vel, ray_time_delta=rtd)
    # upstream gradients on a 2^-12 grid: exact in float32 and small once compressed
    q = lambda shape: (np.round(g.normal(size=shape) * 40.0) / 4096.0).astype(np.float32)
    vr, vd, va = q(rgb.shape), q(dep.shape), q(alp.shape)
    gr = O.eval3d_bwd(means, quats, scales, colors, opac, ro, rd, off, fl, alp, last, vr, vd, va, tsx, tsy,
                      velocity=vel, ray_time_delta=rtd)
    case.update(ray_o=ro, ray_d=rd, rgb=rgb, depth=dep, alpha=alp, last_ids=last, v_rgb=vr, v_depth=vd,
                v_alpha=va)
    for k, v in gr.items():
        case["g_" + k] = v
    return case


def case_pinhole_sh():
    """Rotated, translated pinhole; SH degree 1 colours; regular 16x16 tiles on a ragged image."""
    g = np.random.default_rng(100)
    W, H, n, deg = 72, 40, 500, 1
    q = S._quat_mul(S._axis_angle_quat([0.0, 1.0, 0.0], math.radians(6.0)),
                    S._axis_angle_quat([1.0, 0.0, 0.0], math.radians(-4.0)))
    spec = S.pinhole(W, H, 66.0, 70.0, 35.0, 21.0, q=q, t=[0.15, -0.1, 0.05])
    z = g.uniform(1.5, 12.0, n)
    means = np.stack([g.uniform(-0.7, 0.7, n) * z, g.uniform(-0.45, 0.45, n) * z, z], -1).astype(np.float32)
    scales = np.exp(g.normal(-2.6, 0.45, (n, 3))).astype(np.float32)
    quats = _unit_quats(g, n)
    opac = _sigmoid(g.normal(0.3, 1.5, n))
    sh = np.concatenate([g.normal(0, 0.3, (n, 1, 3)), g.normal(0, 0.08, (n, (deg + 1) ** 2 - 1, 3))], 1)
    sh = sh.astype(np.float32)
    origin = np.array(spec.t, np.float32)
    colors = O.sh_fwd(deg, origin, means, sh)
    flags, radii, m2, dep = O.project_utgs(spec, means, scales, quats, opac, W, H)
    tpg, ids, fl = O.isect_regular(m2, radii, dep, W, H, 16, 16, sort=True)
    _, ids_u, fl_u = O.isect_regular(m2, radii, dep, W, H, 16, 16, sort=False)
    off = O.offset_encode(ids, (W + 15) // 16, (H + 15) // 16)
    case = dict(spec_arrays(spec), tile=np.array([16, 16], np.int32), sh_degree=np.int32(deg), means=means,
                scales=scales, quats=quats, opacity=opac, sh=sh, colors=colors, ut_flags=flags, radii=radii,
                means2d=m2, depths=dep, tiles_per_gauss=tpg, isect_ids=ids, flatten_ids=fl,
                isect_ids_unsorted=ids_u, flatten_ids_unsorted=fl_u, offsets=off)
    composite(case, spec, W, H, 16, 16, means, quats, scales, opac, colors, off, fl, g)
    d_sh, _, d_pos, d_origin = O.sh_bwd(deg, origin, means, sh, case["g_v_colors"])
    case.update(sh_d_coeffs=d_sh, sh_d_positions=d_pos, sh_d_origin=d_origin)
    return case


def case_lidar_phm():
    """Spinning lidar (rolling shutter along azimuth) with phm seam handling, CDIM 2 features."""
    g = np.random.default_rng(200)
    W, n_beams, n, tsx, tsy = 96, 32, 700, 16, 8
    _, beam_v, limits = S.lidar_beams(n_beams)
    spec = S.CameraSpec("lidar", W, n_beams, [1.0, 0.0, 0.0, 0.0], [0.0, 0.0, 0.0], limits, beam_v=beam_v)
    spec.rolling = [0.1, 0.0]
    spec.trigger_time, spec.pose_time = 0.0, 0.05      # seam (u_pose) at mid-sweep
    r = np.exp(g.uniform(math.log(2.0), math.log(40.0), n))
    az = g.uniform(0, 2 * math.pi, n)
    means = np.stack([r * np.cos(az), r * np.sin(az), g.uniform(-1.5, 3.0, n)], -1).astype(np.float32)
    scales = np.exp(g.normal(-1.6, 0.5, (n, 3))).astype(np.float32)
    quats = _unit_quats(g, n)
    opac = _sigmoid(g.normal(0.5, 1.5, n))
    colors = np.stack([g.uniform(0, 1, n), g.normal(0, 1, n)], -1).astype(np.float32)
    flags, radii, m2, dep = O.project_utgs(spec, means, scales, quats, opac, W, n_beams, phm=True)
    elev = beam_v.numpy()[::tsy].astype(np.float32)
    tpg, ids, fl = O.isect_spherical_family("lidar", spec, means, scales, quats, opac, flags, m2, radii, dep, tsx,
                                           tsy, W, n_beams, elev=elev)
    ntw, nth = (W + tsx - 1) // tsx, elev.shape[0]
    off = O.offset_encode(ids, ntw, nth)
    case = dict(spec_arrays(spec), tile=np.array([tsx, tsy], np.int32), elev=elev, means=means, scales=scales,
                quats=quats, opacity=opac, colors=colors, ut_flags=flags, radii=radii, means2d=m2, depths=dep,
                tiles_per_gauss=tpg, isect_ids=ids, flatten_ids=fl, offsets=off)
    return composite(case, spec, W, n_beams, tsx, tsy, means, quats, scales, opac, colors, off, fl, g)


def case_spherical():
    """Static spherical camera, regular angular tiles (exclusive bounds)."""
    g = np.random.default_rng(300)
    W, H, n, tsx, tsy = 80, 32, 500, 16, 16
    spec = S.CameraSpec("spherical", W, H, [1.0, 0.0, 0.0, 0.0], [0.0, 0.0, 0.0],
                        [0.0, 2 * math.pi, -0.6, 1.2])
    r = g.uniform(2.0, 25.0, n)
    az = g.uniform(0, 2 * math.pi, n)
    means = np.stack([r * np.cos(az), r * np.sin(az), g.uniform(-0.25, 0.25, n) * r], -1).astype(np.float32)
    scales = np.exp(g.normal(-1.2, 0.4, (n, 3))).astype(np.float32)
    quats = _unit_quats(g, n)
    opac = _sigmoid(g.normal(0.5, 1.5, n))
    colors = g.uniform(0, 1, (n, 3)).astype(np.float32)
    flags, radii, m2, dep = O.project_utgs(spec, means, scales, quats, opac, W, H, phm=True)
    tpg, ids, fl = O.isect_spherical_family("spherical", spec, means, scales, quats, opac, flags, m2, radii, dep,
                                           tsx, tsy, W, H)
    off = O.offset_encode(ids, W // tsx, H // tsy)
    case = dict(spec_arrays(spec), tile=np.array([tsx, tsy], np.int32), means=means, scales=scales, quats=quats,
                opacity=opac, colors=colors, ut_flags=flags, radii=radii, means2d=m2, depths=dep,
                tiles_per_gauss=tpg, isect_ids=ids, flatten_ids=fl, offsets=off)
    return composite(case, spec, W, H, tsx, tsy, means, quats, scales, opac, colors, off, fl, g)


def case_dynamic():
    """Moving rolling-shutter pinhole and moving Gaussians: point projection, UT with velocity,
    dynamic composite with a per-pixel time delta."""
    g = np.random.default_rng(400)
    W, H, n = 48, 32, 300
    spec = S.pinhole(W, H, 46.0, 46.0, 24.0, 16.0)
    spec.v, spec.w = [1.5, 0.2, -0.4], [0.03, -0.05, 0.1]
    spec.rolling = [0.0, 0.04]
    spec.trigger_time, spec.pose_time = 0.0, 0.02
    z = g.uniform(2.0, 9.0, n)
    means = np.stack([g.uniform(-0.6, 0.6, n) * z, g.uniform(-0.5, 0.5, n) * z, z], -1).astype(np.float32)
    vel = g.normal(0, 0.8, (n, 3)).astype(np.float32)
    scales = np.exp(g.normal(-2.2, 0.4, (n, 3))).astype(np.float32)
    quats = _unit_quats(g, n)
    opac = _sigmoid(g.normal(0.3, 1.5, n))
    colors = g.uniform(0, 1, (n, 3)).astype(np.float32)
    uvdt, pmask = O.projection(spec, means, vel=vel)
    flags, radii, m2, dep = O.project_utgs(spec, means, scales, quats, opac, W, H, vel=vel)
    tpg, ids, fl = O.isect_regular(m2, radii, dep, W, H, 16, 16, sort=True)
    off = O.offset_encode(ids, W // 16, H // 16)
    rtd = _pixel_time_delta(spec, W, H)
    case = dict(spec_arrays(spec), tile=np.array([16, 16], np.int32), means=means, velocity=vel, scales=scales,
                quats=quats, opacity=opac, colors=colors, proj_uvdt=uvdt, proj_mask=pmask, ut_flags=flags,
                radii=radii, means2d=m2, depths=dep, tiles_per_gauss=tpg, isect_ids=ids, flatten_ids=fl,
                offsets=off, ray_time_delta=rtd)
    return composite(case, spec, W, H, 16, 16, means, quats, scales, opac, colors, off, fl, g, vel=vel, rtd=rtd)


CASES = {"pinhole_sh": case_pinhole_sh, "lidar_phm": case_lidar_phm, "spherical": case_spherical,
         "dynamic": case_dynamic}


def main():
    O.build()
    for name, fn in CASES.items():
        case = fn()
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **case)
        print(f"{name}: {os.path.getsize(path) / 1024:.0f} KiB, "
              f"{int(case['isect_ids'].shape[0])} isects, flags {np.bincount(case['ut_flags'], minlength=3)}")


if __name__ == "__main__":
    main()
