"""xsimgs_amd: the xsimgs Gaussian-splatting rasterization hot path on MI355X (gfx950).

``xsimgs_amd._C`` re-exports the reference's native op names (``xsimgs._C``) over hand-written
HIP kernels; ``xsimgs_amd.rendering`` and ``xsimgs_amd.cameras`` mirror the reference's Python
layer (``xsimgs.rendering``, ``xsimgs.cameras.ext``). Importing fails loudly when the native
libraries have not been built: there is no CPU fallback.
"""
import os as _os

_here = _os.path.dirname(_os.path.abspath(__file__))
try:
    import torch as _torch  # noqa: F401  (loads the HIP runtime the extension shares)
    from . import _C  # noqa: F401
except ImportError as _e:  # pragma: no cover - exercised only without a build
    raise ImportError(
        "xsimgs_amd native extension is not built; run `python -c \"import __graft_entry__ as g; g.build()\"` "
        f"from the repository root ({_e})") from _e

from . import rendering, cameras  # noqa: E402,F401
from .rendering import ut_gs_render, ut_gs_tiling, ut_gs_rasterize  # noqa: E402,F401
from .rendering.sh import *  # noqa: E402,F401,F403

LIB_PATH = _os.path.join(_here, "libxsimgs_hip.so")
