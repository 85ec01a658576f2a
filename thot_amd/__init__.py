"""thot_amd — MI355X (gfx950) training-backward kernels behind Nott's API.

The product is libnott_hip.so (HIP kernels + the C ABI in include/nott_hip.h).
`thot_amd.ops` is a thin torch-tensor layer over that ABI; `thot_amd.build`
compiles the library in-tree.  Importing the package does not load the
library; the first op call does, and raises if it is missing.
"""
from . import _abi  # noqa: F401

__all__ = ["_abi", "ops", "build"]
