"""Alias of :mod:`gswarp_amd.methods` under the reference package name."""

from gswarp_amd.methods import *  # noqa: F401,F403
from gswarp_amd.methods import __all__  # noqa: F401
