"""Rasterizer method variants built on the gfx950 pipeline.

Only the Mip-Splatting screen-space filter (``mip_3dgs``) is provided; it is the
standard rasterizer with a filter variance added to every 2D covariance.
"""

from .mip_3dgs import METHOD as MIP_3DGS

__all__ = ["MIP_3DGS"]
