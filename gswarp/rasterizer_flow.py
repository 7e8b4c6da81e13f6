"""Alias of :mod:`gswarp_amd.rasterizer_flow` under the reference module name."""

from gswarp_amd.rasterizer_flow import *  # noqa: F401,F403
from gswarp_amd.rasterizer_flow import __all__  # noqa: F401
