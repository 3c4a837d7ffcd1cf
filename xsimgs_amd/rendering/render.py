"""Frame orchestration: reference src/xsimgs/rendering/render.py:10-187.

``ut_gs_tiling`` runs the UT projection, optional radius masking, tile binning with sort and
the per-tile offsets; ``ut_gs_render`` adds the camera rays and the (static or dynamic)
compositor, in the reference's order.
"""
import torch

from .._C import mask_radii, eval3d_supported_ndims
from .rasterize import ut_gs_rasterize
from .rasterize_dynamic import ut_gs_dynamic_rasterize


def ut_gs_tiling(camera, points, scale, rotation, width: int, height: int, points_velocity=None, opacity=None,
                 packed_particle_mask=None, tile_size_x: int = 16, tile_size_y: int = 16, ut_alpha: float = 0.1,
                 ut_beta: float = 2.0, ut_kappa: float = 0.0, use_phm: bool = None) -> dict:
    with camera._freeze_ctx():
        flags, radii, means2d, depth = camera.ut_gs_projection(
            points=points, points_velocity=points_velocity, scale=scale, rotation=rotation, opacity=opacity,
            width=width, height=height, ut_alpha=ut_alpha, ut_beta=ut_beta, ut_kappa=ut_kappa, use_phm=use_phm)
        if packed_particle_mask is not None:
            mask_radii(packed_particle_mask, radii)
        n_tiles_width = (width + tile_size_x - 1) // tile_size_x
        n_tiles_height = (height + tile_size_y - 1) // tile_size_y
        # the sorted fill writes the tile offsets that isect_offset_encode would compute from its keys, so
        # the keys themselves (read by nothing else here) are not written
        tile_gs_offsets = torch.empty((n_tiles_height, n_tiles_width), dtype=torch.int32, device=points.device)
        tiles_per_gs, isect_ids, flatten_ids = camera.isect_gs_tiles(
            points=points, points_velocity=points_velocity, scale=scale, rotation=rotation, opacity=opacity,
            flags=flags, means2d=means2d, radii=radii, depths=depth, width=width, height=height,
            ut_alpha=ut_alpha, ut_beta=ut_beta, ut_kappa=ut_kappa, tile_size_x=tile_size_x,
            tile_size_y=tile_size_y, sort=True, double_buffer=True, tile_offsets=tile_gs_offsets, keys=False)
    return dict(means2d=means2d, radii=radii, depth=depth, isect_offsets=tile_gs_offsets, flatten_ids=flatten_ids)


def ut_gs_render(camera, points, scale, rotation, opacity, width: int, height: int, colors=None,
                 points_velocity=None, packed_particle_mask=None, tile_size_x: int = 16, tile_size_y: int = 16,
                 ut_alpha: float = 0.1, ut_beta: float = 2.0, ut_kappa: float = 0.0, use_phm: bool = None,
                 ray_o=None, ray_d=None, ray_time_delta=None):
    assert camera.device == points.device, (
        "Camera must be on the same device as gaussian tensors. Given camera on {}, points on {}".format(
            camera.device, points.device))
    if colors is not None:
        assert colors.shape[-1] in eval3d_supported_ndims(), (
            "Color feature dimension = {} is not supported. Supported CDIMs=[{}].".format(
                colors.shape[-1], ', '.join(str(v) for v in eval3d_supported_ndims())))
    with camera._freeze_ctx():
        points = points.contiguous()
        scale = scale.contiguous()
        rotation = rotation.contiguous()
        opacity = opacity.contiguous()
        colors = colors.contiguous() if colors is not None else None
        points_velocity = points_velocity.contiguous() if points_velocity is not None else None
        # rays first (independent of the tiling): they run on the GPU ahead of the tiling's one
        # host readback instead of after it
        if ray_o is None or ray_d is None:
            ray_o, ray_d = camera.camera_rays(width=width, height=height, normalized_rays=True, return_origins=True,
                                              world_space=True)
        tile_data = ut_gs_tiling(camera=camera, points=points, scale=scale, rotation=rotation, width=width,
                                 height=height, points_velocity=points_velocity, opacity=opacity,
                                 packed_particle_mask=packed_particle_mask, tile_size_x=tile_size_x,
                                 tile_size_y=tile_size_y, ut_alpha=ut_alpha, ut_beta=ut_beta, ut_kappa=ut_kappa,
                                 use_phm=use_phm)
        is_scene_static = points_velocity is None
        kwargs = dict(positions=points, rotation=rotation, scale=scale, density=opacity, colors=colors, ray_o=ray_o,
                      ray_d=ray_d, isect_offsets=tile_data['isect_offsets'], flatten_ids=tile_data['flatten_ids'],
                      tile_size_x=tile_size_x, tile_size_y=tile_size_y)
        if is_scene_static:
            color, depth, alpha = ut_gs_rasterize(**kwargs)
        else:
            if ray_time_delta is None:
                ray_time_delta = camera.image_time_delta(ray_o)
            color, depth, alpha = ut_gs_dynamic_rasterize(**kwargs, velocity=points_velocity,
                                                          ray_time_delta=ray_time_delta)
    meta = dict(radii=tile_data['radii'], width=width, height=height)
    return color, depth, alpha, meta
