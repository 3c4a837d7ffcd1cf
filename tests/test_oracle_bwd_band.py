"""Pin of the oracle's compositor backward in the alpha band between its two clamps (CPU only).

The forward clamps alpha at 0.999 (eval3d_fwd.cu:127) and the backward at 0.99 (eval3d_bwd.cu:38,
202), and the backward drops the geometry and opacity gradients of a pair with op * vis > 0.99
(:243). Finite differences cannot check this deliberate non-derivative, so it is pinned by a closed
form derived by hand from those rules: one pixel whose ray passes through Gaussian A (alpha 0.5) and
then 0.01 m beside the centre of Gaussian B (op * vis = 0.9999 exp(-0.005) = 0.99491, inside the
band). The forward composites B unclamped; the backward replays with alpha_B = 0.99:

  T_B = T_final / (1 - 0.99),  fac_B = 0.99 T_B,  v_colors_B = fac_B v_rgb,  every other gradient of B 0;
  T_A = T_B / (1 - 0.5),       fac_A = 0.5 T_A,   v_colors_A = fac_A v_rgb,
  dL/dalpha_A = sum_c (rgb_A T_A - 2 fac_B rgb_B) v_rgb + (3 T_A - 2 fac_B 5) v_depth + 2 T_final v_alpha
  (grad_alpha, eval3d_bwd.cu:42-63, with the depth buffer fac_B t_B and t_B = 5);
  v_opacity_A = vis_A dL/dalpha_A with vis_A = 1 on its centre; v_means_A = (0, 0, fac_A v_depth) from
  the hit distance (A on the ray: no alpha term); A is isotropic with its centre on the ray, so its
  hit distance and alpha do not move with its rotation or scale.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


def _band_scene():
    means = np.array([[0.0, 0.0, 3.0], [0.01, 0.0, 5.0]])
    scales = np.array([[0.2, 0.2, 0.2], [0.1, 0.1, 0.1]])
    quats = np.array([[1.0, 0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 0.0]])
    opac = np.array([0.5, 0.9999])
    rgb = np.array([[0.2, 0.5, 0.9], [0.7, 0.1, 0.3]])
    ro = np.zeros((1, 1, 3))
    rd = np.array([[[0.0, 0.0, 1.0]]])
    off = np.zeros((1, 1), np.int32)
    fl = np.array([0, 1], np.int32)
    return means, quats, scales, rgb, opac, ro, rd, off, fl


@pytest.mark.parametrize("prec,tol", [("f64", 1e-12), ("f32", 2e-6)])
def test_bwd_clamp_band_closed_form(prec, tol):
    means, quats, scales, rgb, opac, ro, rd, off, fl = _band_scene()
    vis_b = math.exp(-0.5 * (0.01 / 0.1) ** 2)
    araw_b = 0.9999 * vis_b
    assert 0.99 < araw_b < 0.999
    rgb_o, dep_o, alp_o, last = O.eval3d_fwd(means, quats, scales, rgb, opac, ro, rd, off, fl, 16, 16, prec=prec)
    T_final = 0.5 * (1 - araw_b)
    # forward: B composited unclamped
    assert abs(alp_o[0, 0] - (1 - T_final)) <= tol
    assert abs(dep_o[0, 0] - (0.5 * 3.0 + 0.5 * araw_b * 5.0)) <= 10 * tol
    assert np.allclose(rgb_o[0, 0], 0.5 * rgb[0] + 0.5 * araw_b * rgb[1], atol=tol)
    assert last[0, 0] == 1
    v_rgb = np.array([[[0.3, -0.7, 0.4]]])
    v_d = np.array([[0.25]])
    v_a = np.array([[-0.6]])
    g = O.eval3d_bwd(means, quats, scales, rgb, opac, ro, rd, off, fl, np.asarray(alp_o), last, v_rgb, v_d, v_a,
                     16, 16, prec=prec)
    T_fin = 1.0 - float(alp_o[0, 0])    # the backward starts from the rendered alpha
    T_b = T_fin / (1 - 0.99)
    fac_b = 0.99 * T_b
    T_a = T_b / (1 - 0.5)
    fac_a = 0.5 * T_a
    vr, vd, va = v_rgb[0, 0], v_d[0, 0], v_a[0, 0]
    dalpha_a = float(np.sum((rgb[0] * T_a - 2 * fac_b * rgb[1]) * vr) + (3.0 * T_a - 2 * fac_b * 5.0) * vd
                     + 2 * T_fin * va)
    expect = dict(
        v_colors=np.array([vr * fac_a, vr * fac_b]),
        v_opacity=np.array([dalpha_a, 0.0]),
        v_means=np.array([[0.0, 0.0, fac_a * vd], [0.0, 0.0, 0.0]]),
        v_quats=np.zeros((2, 4)),
        v_scales=np.zeros((2, 3)),
    )
    for k, e in expect.items():
        print(prec, k, g[k].tolist())
        assert np.allclose(g[k], e, rtol=50 * tol, atol=tol), (k, g[k], e)
    # B's gradients are exactly zero (gated), not merely small
    for k in ("v_opacity", "v_means", "v_quats", "v_scales"):
        assert not np.any(g[k][1]), k
    # and they are not the derivative: an unclamped replay would weight B's colour by its visibility
    assert abs(fac_b - araw_b * 0.5) > 0.1
