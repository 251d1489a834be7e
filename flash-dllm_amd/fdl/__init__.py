"""MI355X-native Flash-Cache hot path of Flash-dLLM: host side.

    fdl.lib       ctypes binding of libfdl.so (include/fdl.h)
    fdl.ops       torch-facing wrappers of the C-ABI entry points
    fdl.schedule  block-table / work-list building
"""
from . import lib, ops, schedule  # noqa: F401
from .lib import FdlError  # noqa: F401
