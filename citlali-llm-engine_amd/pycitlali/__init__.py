"""Python side of the MI355X Citlali decode hot path.

The compute lives in libcitlali_hip.so (gfx950 kernels behind the C ABI of
include/citlali_hip.h); this package only binds it with ctypes, manages
device buffers and generates seeded synthetic inputs.
"""
from . import _lib, device, dtype, synth  # noqa: F401
from ._lib import CitlaliError, check, last_error, load  # noqa: F401
from .device import DeviceArray, Event, synchronize  # noqa: F401
