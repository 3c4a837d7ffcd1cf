"""Autograd wrappers and frame orchestration (reference src/xsimgs/rendering)."""
from .activate import activate_gaussians
from .render import ut_gs_render, ut_gs_tiling
from .rasterize import ut_gs_rasterize, ut_gs_rasterize_batched
from .rasterize_dynamic import ut_gs_dynamic_rasterize
from .sh import *  # noqa: F401,F403
