"""apply_grad_mask: gradients only for inputs that require them (toast.ops.ext.apply_grad_mask,
used by the reference at rendering/rasterize.py:72 and rendering/sh.py:42)."""


def apply_grad_mask(ctx, grads):
    return tuple(g if (i < len(ctx.needs_input_grad) and ctx.needs_input_grad[i]) else None
                 for i, g in enumerate(grads))
