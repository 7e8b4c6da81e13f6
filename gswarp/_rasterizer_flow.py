"""Alias of :mod:`gswarp_amd._rasterizer_flow` (the raw flow ABI) under the reference module name."""

from gswarp_amd._rasterizer_flow import *  # noqa: F401,F403
from gswarp_amd._rasterizer_flow import __all__  # noqa: F401
