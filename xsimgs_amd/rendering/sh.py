"""SphericalHarmonicsFused: reference src/xsimgs/rendering/sh.py:11-71."""
import torch

from .._C import spherical_harmonics_fused_fwd, spherical_harmonics_fused_bwd
from ._grad import apply_grad_mask

__all__ = ["SphericalHarmonicsFused", "spherical_harmonics_fused", "sh_degree_to_bands",
           "sh_degree_to_specular_dim", "rgb_to_sh0", "sh0_to_rgb"]


class SphericalHarmonicsFused(torch.autograd.Function):
    @staticmethod
    def forward(ctx, coeffs, positions, origin, degree_to_use: int, mask=None, layout_3kn: bool = False,
                coeffs_dc=None):
        ctx.layout_3kn = layout_3kn
        ctx.degree_to_use = degree_to_use
        ctx.save_for_backward(origin, positions, coeffs, mask, coeffs_dc)
        return spherical_harmonics_fused_fwd(degree_to_use, origin, positions, coeffs, mask, layout_3kn, coeffs_dc)

    @staticmethod
    def backward(ctx, grad_out):
        origin, positions, coeffs, mask, coeffs_dc = ctx.saved_tensors
        # the origin gradient (a sum over every Gaussian) only when the origin needs one
        d_coeffs, d_coeffs_dc, d_positions, d_origin = spherical_harmonics_fused_bwd(
            ctx.degree_to_use, origin, positions, coeffs, mask, ctx.layout_3kn, grad_out.contiguous(), coeffs_dc,
            origin_grad=ctx.needs_input_grad[2])
        # order of the forward inputs: coeffs, positions, origin, degree_to_use, mask, layout_3kn, coeffs_dc
        return apply_grad_mask(ctx, (d_coeffs, d_positions, d_origin, None, None, None, d_coeffs_dc))


def spherical_harmonics_fused(coeffs, positions, origin, degree_to_use: int, mask=None, layout_3kn: bool = False,
                              coeffs_dc=None):
    return SphericalHarmonicsFused.apply(coeffs, positions, origin, degree_to_use, mask, layout_3kn, coeffs_dc)


def sh_degree_to_bands(degree: int):
    return (degree + 1) ** 2


def sh_degree_to_specular_dim(degree: int):
    """Number of dimensions used by SH of deg [1...degree], inclusive"""
    return 3 * (sh_degree_to_bands(degree) - 1)


def rgb_to_sh0(rgb: torch.Tensor) -> torch.Tensor:
    C0 = 0.28209479177387814
    return (rgb - 0.5) / C0


def sh0_to_rgb(sh: torch.Tensor) -> torch.Tensor:
    C0 = 0.28209479177387814
    return sh * C0 + 0.5
