"""MI355X (gfx950) numeric execution backend for the kernels the Wafer
compiler emits: hand-written HIP kernels behind the C ABI in
include/wafer_hip.h, reached from Python through `backend`.
"""
from . import backend  # noqa: F401

__all__ = ["backend"]
