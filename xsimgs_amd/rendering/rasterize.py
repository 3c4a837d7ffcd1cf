"""UTGSRasterize: autograd contract of reference src/xsimgs/rendering/rasterize.py:6-100, and its
batched-camera extension UTGSRasterizeBatched."""
import torch

from .._C import (rasterize_eval3d_fwd, rasterize_eval3d_bwd, rasterize_eval3d_fwd_batched,
                  rasterize_eval3d_bwd_batched)
from ._grad import apply_grad_mask, tile_work_buffer


class UTGSRasterize(torch.autograd.Function):
    @staticmethod
    def forward(ctx, positions, rotation, scale, density, colors, ray_o, ray_d, isect_offsets, flatten_ids,
                tile_size_x: int, tile_size_y: int):
        height, width = ray_o.shape[:2]
        out_rgb, out_depth, out_alpha, last_ids = rasterize_eval3d_fwd(
            means=positions, quats=rotation, scales=scale, opacities=density.view(1, -1),
            colors=colors.unsqueeze(0) if colors is not None else None, ray_origs=ray_o, ray_dirs=ray_d,
            image_width=width, image_height=height, tile_size_width=tile_size_x,
            tile_size_height=tile_size_y, tile_offsets=isect_offsets, flatten_ids=flatten_ids,
            tile_work=tile_work_buffer(ctx, isect_offsets))
        ctx.tile_size_x = tile_size_x
        ctx.tile_size_y = tile_size_y
        ctx.save_for_backward(positions, rotation, scale, density, colors, ray_o, ray_d, isect_offsets,
                              flatten_ids, out_alpha, last_ids)
        return out_rgb, out_depth, out_alpha

    @staticmethod
    def backward(ctx, grad_rgb, grad_depth, grad_alpha):
        (positions, rotation, scale, density, colors, ray_o, ray_d, isect_offsets, flatten_ids, out_alpha,
         last_ids) = ctx.saved_tensors
        # v_points, v_quat, v_scale, v_opacity, v_colors, v_ray_o, v_ray_d
        grads = rasterize_eval3d_bwd(
            positions, scale, rotation, density, colors, ray_o, ray_d, ctx.tile_size_x, ctx.tile_size_y,
            isect_offsets, flatten_ids, out_alpha, last_ids,
            grad_rgb.contiguous() if grad_rgb is not None else None, grad_depth.contiguous(),
            grad_alpha.contiguous(),
            ctx.needs_input_grad[5] or ctx.needs_input_grad[6], tile_work=ctx.tile_work)
        return apply_grad_mask(ctx, list(grads) + [None, None, None, None])


def ut_gs_rasterize(positions, rotation, scale, density, colors, ray_o, ray_d, isect_offsets, flatten_ids,
                    tile_size_x: int, tile_size_y: int):
    return UTGSRasterize.apply(positions, rotation, scale, density, colors, ray_o, ray_d, isect_offsets,
                               flatten_ids, tile_size_x, tile_size_y)


class UTGSRasterizeBatched(torch.autograd.Function):
    """C cameras over one scene in one compositor launch per pass (an extension of this build; the
    reference composites one camera per call). Rays are [C, H, W, 3], offsets [C, th, tw] and
    flatten ids cam * N + gaussian from isect_regular_tiles_batched; colours are per camera
    [C, N, ch] or shared by every camera [N, ch], whose gradient then sums over the cameras. Each
    camera's images equal a single-camera call's on that camera's tiles."""

    @staticmethod
    def forward(ctx, positions, rotation, scale, density, colors, ray_o, ray_d, isect_offsets, flatten_ids,
                tile_size_x: int, tile_size_y: int):
        height, width = ray_o.shape[1:3]
        out_rgb, out_depth, out_alpha, last_ids = rasterize_eval3d_fwd_batched(
            means=positions, quats=rotation, scales=scale, opacities=density, colors=colors, ray_origs=ray_o,
            ray_dirs=ray_d, image_width=width, image_height=height, tile_size_width=tile_size_x,
            tile_size_height=tile_size_y, tile_offsets=isect_offsets, flatten_ids=flatten_ids,
            tile_work=tile_work_buffer(ctx, isect_offsets))
        ctx.tile_size_x = tile_size_x
        ctx.tile_size_y = tile_size_y
        ctx.save_for_backward(positions, rotation, scale, density, colors, ray_o, ray_d, isect_offsets,
                              flatten_ids, out_alpha, last_ids)
        return out_rgb, out_depth, out_alpha

    @staticmethod
    def backward(ctx, grad_rgb, grad_depth, grad_alpha):
        (positions, rotation, scale, density, colors, ray_o, ray_d, isect_offsets, flatten_ids, out_alpha,
         last_ids) = ctx.saved_tensors
        grads = rasterize_eval3d_bwd_batched(
            positions, scale, rotation, density, colors, ray_o, ray_d, ctx.tile_size_x, ctx.tile_size_y,
            isect_offsets, flatten_ids, out_alpha, last_ids,
            grad_rgb.contiguous() if grad_rgb is not None else None, grad_depth.contiguous(),
            grad_alpha.contiguous(), ray_grads=ctx.needs_input_grad[5] or ctx.needs_input_grad[6],
            tile_work=ctx.tile_work)
        # v_points, v_quat, v_scale, v_opacity, v_colors, v_ray_o, v_ray_d (static: no velocity terms)
        return apply_grad_mask(ctx, list(grads[:7]) + [None, None, None, None])


def ut_gs_rasterize_batched(positions, rotation, scale, density, colors, ray_o, ray_d, isect_offsets, flatten_ids,
                            tile_size_x: int, tile_size_y: int):
    return UTGSRasterizeBatched.apply(positions, rotation, scale, density, colors, ray_o, ray_d, isect_offsets,
                                      flatten_ids, tile_size_x, tile_size_y)
