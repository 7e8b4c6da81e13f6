"""Import alias so existing ``import gswarp`` code runs on the gfx950 build.

Re-exports the public surface of :mod:`gswarp_amd` under the reference's
module names (``gswarp``, ``gswarp.rasterizer``, ``gswarp.rasterizer_flow``).
"""

from gswarp_amd import *  # noqa: F401,F403
from gswarp_amd import __version__, distCUDA2, fused_ssim  # noqa: F401
from gswarp_amd.rasterizer import __all__ as _rasterizer_all

__all__ = list(_rasterizer_all) + ["fused_ssim", "distCUDA2"]
