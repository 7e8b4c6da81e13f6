"""Alias of :mod:`gswarp_amd.methods.mip_3dgs` under the reference module name."""

from gswarp_amd.methods.mip_3dgs import *  # noqa: F401,F403
from gswarp_amd.methods.mip_3dgs import __all__  # noqa: F401
