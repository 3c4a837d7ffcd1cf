"""Pin of the oracle's phase-modelled UT (orc_project_utgs_phm; ut_phm_kernels.h:13-114), CPU only.

The projection of each mode is restated here from the geometry in float64 numpy, independently of the
oracle's code: a point at azimuth phi = atan2(-x, -y) + pi (spherical.h:24-31) maps to
u = (phi - phi_min) / phi_range, and the NegativeDelta / PositiveDelta modes unwrap u by one turn
(2 pi / phi_range) on the side of u_pose their shutter direction selects (spherical.h:109-125); the UT
then averages seven sigma points (ut_kernels.h:52-137, 140-184). Gaussians are placed where the flag
and the stored side follow from the geometry, by hand:

* far from both seams: only the Central UT is compact and on screen -> flag 1, Central outputs;
* straddling the image seam (phi = phi_min): Central spreads over the turn (u_distance > u_pi), both
  unwrapped modes are compact -> flag 2 with the NegativeDelta outputs, whose mean lies one image
  width from the PositiveDelta one (so a left / right swap would fail);
* straddling u_pose: Central compact, both unwrapped modes split -> flag 1, Central;
* a footprint crossing the image edge while its sigma points do not: all three compact and on screen
  -> flag 2, NegativeDelta;
* on a half-turn camera (phi_range = pi, one turn = 2 in u), a Gaussian straddling phi_min: Central
  spreads over the turn, NegativeDelta leaves the projection's margin, PositiveDelta compact -> the reference's
  last branch (ut_phm_kernels.h:105-113) stores the side that is not compact (`use_left =
  result_left != 1`): flag 1 with the NegativeDelta mean, whose failed projection leaves the
  covariance unset in the reference; here it is zero, so the radii are (0, 0).

Each case runs with a global shutter (u_pose = 0.5, spherical.h:111-112), a positive and a negative
rolling time (u_pose from the pose and trigger times). The cameras are static, so the shutter only
moves u_pose.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from xsimgs_amd import synthetic as S

W, H = 2048, 64
ALPHA, BETA, KAPPA = 0.1, 2.0, 0.0
TIMINGS = {  # rolling time (u), pose time - trigger time -> u_pose
    "global": (0.0, 0.0),
    "rolling_pos": (0.1, 0.03),     # u_pose 0.3
    "rolling_neg": (-0.1, -0.07),   # u_pose 0.7
}


def _spec(timing, phi_range=2 * math.pi, width=W):
    roll, dt = TIMINGS[timing]
    limits = [0.0, phi_range, 0.35, -0.7]   # theta from +0.35 down to -0.35 rad over the rows
    return S.CameraSpec("spherical", width, H, [1.0, 0.0, 0.0, 0.0], [0.0, 0.0, 0.0], limits,
                        rolling=[roll, 0.0], trigger_time=0.0, pose_time=dt)


def _u_pose(spec):
    roll = spec.rolling[0]
    return (spec.pose_time - spec.trigger_time) / roll if abs(roll) > 0 else 0.5


def _rot(q):
    w, x, y, z = np.asarray(q, np.float64) / np.linalg.norm(q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def _ut_mode(spec, mu, q, s, op, mode):
    """One mode's UT from the geometry: (valid, mean2d px, radii px, depth, u_distance px)."""
    phi_min, phi_range, th_min, th_range = spec.impl
    width, height = spec.width, spec.height
    lam = ALPHA ** 2 * (3 + KAPPA) - 3
    wm0, wi = lam / (3 + lam), 1 / (2 * (3 + lam))
    wc0 = wm0 + (1 - ALPHA ** 2 + BETA)
    R = _rot(q)
    d = [R[:, k] * s[k] * math.sqrt(3 + lam) for k in range(3)]
    pts = [np.asarray(mu, np.float64)]
    for i in range(6):
        pts.append(pts[0] + (1.0 if i % 2 == 0 else -1.0) * d[i // 2])
    u_pose, turn = _u_pose(spec), 2 * math.pi / abs(phi_range)
    px, valid = [], True
    for p in pts:
        r = np.linalg.norm(p)
        u = (math.atan2(-p[0], -p[1]) + math.pi - phi_min) / phi_range
        v = (math.asin(p[2] / r) - th_min) / th_range
        if spec.rolling[0] > 0:
            u = u - turn if (mode == "negative" and u > u_pose) else u
            u = u + turn if (mode == "positive" and u < u_pose) else u
        else:
            u = u + turn if (mode == "negative" and u < u_pose) else u
            u = u - turn if (mode == "positive" and u > u_pose) else u
        if not (-1.0 <= u <= 2.0 and -1.0 <= v <= 2.0):   # max_margin = 1 (projection_kernels.h:240-247)
            valid = False
            u = v = 0.0                                   # a failed point contributes zeros
        px.append(np.array([u * width, v * height]))
    depth = np.linalg.norm(pts[0])
    mean = wm0 * px[0] + wi * sum(px[1:])
    if not valid:
        return False, mean, np.zeros(2), depth, 0.0
    u_dist = max(p[0] for p in px) - min(p[0] for p in px)
    cov = wc0 * np.outer(px[0] - mean, px[0] - mean) + wi * sum(np.outer(p - mean, p - mean) for p in px[1:])
    ok = np.linalg.det(cov) > 0 and cov[0, 0] >= 0 and cov[1, 1] >= 0
    ext = min(3.33, math.sqrt(2 * math.log(op * 255.0)))
    radii = ext * np.sqrt(np.maximum(np.diag(cov), 0.0))
    on = not (mean[0] + radii[0] < 0 or width < mean[0] - radii[0]) and \
        not (mean[1] + radii[1] < 0 or height < mean[1] - radii[1])
    return bool(ok and on), mean, radii, depth, u_dist


def _at(phi, rho=10.0, z=0.0):
    """A point at azimuth phi, rounded to the float32 value both sides receive."""
    return np.array([rho * math.sin(phi), rho * math.cos(phi), z], np.float32).astype(np.float64)


def seam_cases(timing):
    """The constructed Gaussians of one timing: list of (name, spec, mu, quat, scale, op, flag, side)."""
    spec = _spec(timing)
    u_pose = _u_pose(spec)
    q = [1.0, 0.0, 0.0, 0.0]
    small = [0.05, 0.05, 0.05]
    far_u = 0.6 if u_pose < 0.5 else 0.25
    cases = [
        ("far", spec, _at(2 * math.pi * far_u), q, small, 0.8, 1, "central"),
        ("image_seam", spec, _at(2 * math.pi - 0.0015), q, [0.1, 0.1, 0.1], 0.8, 2, "negative"),
        ("u_pose", spec, _at(2 * math.pi * u_pose + 0.0003), q, [0.1, 0.1, 0.1], 0.8, 1, "central"),
        # sigma points ~0.3 px apart, 2 px left of the edge, radius ~5 px: only the footprint crosses
        ("edge_footprint", spec, _at(2 * math.pi * (1 - 2.0 / W)), q, [0.046, 0.046, 0.046], 0.8, 2, "negative"),
    ]
    half = _spec(timing, phi_range=math.pi, width=1024)
    if timing == "global":
        cases.append(("half_turn_one_sided", half, _at(2 * math.pi - 0.0015), q, [0.1, 0.1, 0.1], 0.8, 1,
                      "negative"))
    return cases


@pytest.mark.parametrize("timing", list(TIMINGS))
def test_phm_seam_selection(timing):
    for name, spec, mu, q, s, op, flag, side in seam_cases(timing):
        modes = {m: _ut_mode(spec, mu, q, s, op, m) for m in ("central", "negative", "positive")}
        u_pi = math.pi * spec.width / abs(spec.impl[1])
        res = {m: int(v[0]) * (int(v[4] > u_pi) + 1) for m, v in modes.items()}
        f, r, m2, d = O.project_utgs(spec, mu[None].astype(np.float32), np.array([s], np.float32),
                                     np.array([q], np.float32), np.array([op], np.float32), spec.width, spec.height,
                                     phm=True, prec="f64")
        print(timing, name, "modes", res, "oracle flag", int(f[0]), "mean", m2[0], "radii", r[0])
        assert int(f[0]) == flag, (timing, name, res)
        v = modes[side]
        assert np.allclose(m2[0], v[1], rtol=1e-9, atol=1e-7), (timing, name)
        assert np.allclose(r[0], v[2], rtol=1e-7, atol=1e-9), (timing, name)
        assert abs(d[0] - v[3]) <= 1e-9 * v[3], (timing, name)
        if flag == 2:   # the two unwrapped modes are a turn apart: a swapped side would be caught
            assert abs(modes["negative"][1][0] - modes["positive"][1][0]) > 0.5 * spec.width
            assert res["negative"] == 1 and res["positive"] == 1
        if name == "far":   # equal to the plain (Central) UT projection
            f0, r0, m0, d0 = O.project_utgs(spec, mu[None].astype(np.float32), np.array([s], np.float32),
                                            np.array([q], np.float32), np.array([op], np.float32), spec.width,
                                            spec.height, prec="f64")
            assert int(f0[0]) == 1 and np.allclose(m0, m2) and np.allclose(r0, r) and np.allclose(d0, d)
        if name == "half_turn_one_sided":
            assert res == {"central": 2, "negative": 0, "positive": 1}
            assert np.all(r[0] == 0.0)
