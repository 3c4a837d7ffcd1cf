"""The caller's parameter activations as one fused op each way: scales = exp(log_scales), opacities =
sigmoid(opacity_logits). An extension of this build: the reference's render takes activated scales and
opacities (src/xsimgs/rendering/render.py:85-96) and its callers apply torch.exp / torch.sigmoid
themselves, one launch each, and autograd adds a launch per gradient. The values and gradients here are
torch's, bit for bit (the same float expressions), in one launch forward and one backward."""
import torch

from .. import _C


class _Activate(torch.autograd.Function):
    @staticmethod
    def forward(ctx, log_scales, opacity_logits):
        ctx.set_materialize_grads(False)
        scales, opacities = _C.activate_fwd(log_scales.contiguous(), opacity_logits.contiguous())
        ctx.save_for_backward(scales, opacities)
        return scales, opacities

    @staticmethod
    def backward(ctx, v_scales, v_opacities):
        scales, opacities = ctx.saved_tensors
        if v_scales is None or not ctx.needs_input_grad[0]:
            v_scales = None
        if v_opacities is None or not ctx.needs_input_grad[1]:
            v_opacities = None
        if v_scales is None and v_opacities is None:
            return None, None
        return _C.activate_bwd(scales, opacities, None if v_scales is None else v_scales.contiguous(),
                            None if v_opacities is None else v_opacities.contiguous())


def activate_gaussians(log_scales: torch.Tensor, opacity_logits: torch.Tensor):
    """(exp(log_scales), sigmoid(opacity_logits)); log_scales holds three values per opacity logit
    ([N, 3] and [N] or [N, 1]), float32 on the GPU."""
    return _Activate.apply(log_scales, opacity_logits)
