"""Alias of :mod:`gswarp_amd.rasterizer` under the reference module name."""

from gswarp_amd.rasterizer import *  # noqa: F401,F403
from gswarp_amd.rasterizer import __all__  # noqa: F401
