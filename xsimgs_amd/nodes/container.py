"""Rigid per-instance copy of Gaussians into the frame's buffers and the packed instance mask:
reference src/xsimgs/nodes/container.py (the autograd function over copy_gs_rigid_transform_{fwd,bwd},
its torch twin, and packed_mask_from_instances). Quaternions are (w, x, y, z)."""
import torch

from .._C import copy_gs_rigid_transform_bwd, copy_gs_rigid_transform_fwd, packed_mask_from_instances


def _grad_mask(ctx, grads):
    """None for every input that does not need a gradient (toast's apply_grad_mask)."""
    return tuple(g if need else None for g, need in zip(grads, ctx.needs_input_grad))


class RigidTransformAndPut(torch.autograd.Function):
    """container.py:14-88: writes the transformed Gaussians into the output buffers in place and
    returns them; the buffers' incoming gradient passes through to the buffers unchanged."""

    @staticmethod
    def forward(ctx, positions, rotations, instance_id, inst_q, inst_t, inst_v, inst_w, inst_mask, out_positions,
                out_rotation, out_velocity, out_mask, buffer_offset, per_instance_offsets, gs_inst_offsets):
        copy_gs_rigid_transform_fwd(positions, rotations, instance_id, inst_q, inst_t, inst_v, inst_w, inst_mask,
                                    out_positions, out_rotation, out_velocity, out_mask, buffer_offset,
                                    per_instance_offsets, gs_inst_offsets)
        ctx.buffer_offset = buffer_offset
        ctx.save_for_backward(positions, rotations, instance_id, inst_q, inst_w, inst_mask, per_instance_offsets,
                              gs_inst_offsets)
        return out_positions, out_rotation, out_velocity

    @staticmethod
    def backward(ctx, v_positions, v_rotation, v_velocity):
        positions, rotations, instance_id, inst_q, inst_w, inst_mask, per_inst, gs_off = ctx.saved_tensors
        g_pos, g_rot, g_q, g_t, g_v, g_w = copy_gs_rigid_transform_bwd(
            positions, rotations, instance_id, inst_q, inst_w, inst_mask, ctx.buffer_offset, per_inst, gs_off,
            v_positions, v_rotation, v_velocity)
        return _grad_mask(ctx, (g_pos, g_rot, None, g_q, g_t, g_v, g_w, None, v_positions, v_rotation, v_velocity,
                                None, None, None, None))


def rigid_transform_and_put(positions, rotations, instance_id, inst_q, inst_t, inst_v, inst_w, inst_mask,
                            out_positions=None, out_rotation=None, out_velocity=None, out_mask=None,
                            buffer_offset: int = 0, per_instance_offsets=None, gs_inst_offsets=None):
    """container.py:91-141: positions [N, 3], rotations [N, 4], instance_id int32 [N], instance poses
    inst_q [K, 4], inst_t, inst_v, inst_w [K, 3], inst_mask bool [K]; output buffers [B, ...]
    (allocated as zeros of the inputs' size when not given). Returns the four buffers."""
    if out_positions is None:
        out_positions = torch.zeros_like(positions.detach())
    if out_rotation is None:
        out_rotation = torch.zeros_like(rotations.detach())
    if out_velocity is None:
        out_velocity = torch.zeros_like(positions.detach())
    if out_mask is None:
        out_mask = torch.zeros_like(positions.detach()[..., 0], dtype=torch.bool)
    out_positions, out_rotation, out_velocity = RigidTransformAndPut.apply(
        positions, rotations, instance_id, inst_q, inst_t, inst_v, inst_w, inst_mask, out_positions, out_rotation,
        out_velocity, out_mask, buffer_offset, per_instance_offsets, gs_inst_offsets)
    return out_positions, out_rotation, out_velocity, out_mask


def _quat_mul(a, b):
    aw, av = a[..., :1], a[..., 1:]
    bw, bv = b[..., :1], b[..., 1:]
    return torch.cat([aw * bw - (av * bv).sum(-1, keepdim=True),
                      aw * bv + bw * av + torch.cross(av, bv, dim=-1)], -1)


def _quat_rotate(q, p):
    w, u = q[..., :1], q[..., 1:]
    uv = torch.cross(u, p, dim=-1)
    return p + 2.0 * (w * uv + torch.cross(u, uv, dim=-1))


def rigid_transform_and_put_torch(positions, rotations, instance_id, inst_q, inst_t, inst_v, inst_w, inst_mask,
                                  out_positions, out_rotation, out_velocity, out_mask, buffer_offset: int,
                                  per_instance_offsets=None, gs_inst_offsets=None):
    """container.py:144-197: the same copy written with torch indexing (any device, autograd by torch)."""
    if out_positions is None:
        out_positions = torch.zeros_like(positions.detach())
        out_rotation = torch.zeros_like(rotations.detach())
        out_velocity = torch.zeros_like(positions.detach())
        out_mask = torch.zeros_like(positions.detach()[..., 0], dtype=torch.bool)
    ids = instance_id.long()
    if per_instance_offsets is not None and gs_inst_offsets is not None:
        out_slice = buffer_offset + gs_inst_offsets.long() + per_instance_offsets.long()[ids]
    else:
        out_slice = torch.arange(buffer_offset, buffer_offset + len(positions), device=positions.device)
    keep = inst_mask[ids].nonzero().view(-1)
    out_slice = out_slice[keep]
    ids_k = ids[keep]
    q = inst_q[ids_k]
    p_rot = _quat_rotate(q, positions[keep])
    out_positions[out_slice] = p_rot + inst_t[ids_k]
    out_rotation[out_slice] = _quat_mul(q, rotations[keep])
    if out_velocity is not None:
        out_velocity[out_slice] = inst_v[ids_k] + torch.cross(inst_w[ids_k], p_rot, dim=-1)
    if out_mask is not None:
        out_mask[out_slice] = True
    return out_positions, out_rotation, out_velocity, out_mask


__all__ = ["RigidTransformAndPut", "rigid_transform_and_put", "rigid_transform_and_put_torch",
           "packed_mask_from_instances"]
