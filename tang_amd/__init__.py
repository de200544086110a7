"""tang_amd: MI355X (gfx950) backend for tang's quantized-inference decode path.

The product is the C-ABI library libtang_hip.so (include/tang_hip.h); this
package builds it (build.py) and binds it for Python callers (capi.py).
"""
from . import capi  # noqa: F401
from .capi import HipComputeDevice, TangHipError  # noqa: F401
