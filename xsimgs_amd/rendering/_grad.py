"""apply_grad_mask: gradients only for inputs that require them (toast.ops.ext.apply_grad_mask,
used by the reference at rendering/rasterize.py:72 and rendering/sh.py:42); tile_work_buffer: the
compositor forward's per-tile work estimates for its backward (an extension of this build)."""
import torch


def apply_grad_mask(ctx, grads):
    return tuple(g if (i < len(ctx.needs_input_grad) and ctx.needs_input_grad[i]) else None
                 for i, g in enumerate(grads))


def tile_work_buffer(ctx, isect_offsets):
    """An int32 buffer of one value per (camera, tile) that the compositor forward fills with the
    backward's work estimates (kept on ctx for the backward, which then skips a pass over the last
    ids); None when no input needs a gradient."""
    ctx.tile_work = None
    if any(ctx.needs_input_grad):
        ctx.tile_work = torch.empty(isect_offsets.numel(), dtype=torch.int32, device=isect_offsets.device)
    return ctx.tile_work
