"""Alias of :mod:`gswarp_amd._rasterizer` (the raw ABI) under the reference module name."""

from gswarp_amd._rasterizer import *  # noqa: F401,F403
from gswarp_amd._rasterizer import __all__  # noqa: F401
