"""vearo_amd -- MI355X (gfx950) backend for vearo's fused layer kernels.

The product is libvearo_hip.so (C ABI in include/vearo_hip.h): hand-written
gfx950 kernels in one code object loaded with hipModuleLoadData, a caching
arena over hipMalloc, and entry points that replace the hot slots of vearo's
BackendOps table. `vearo_amd.ops` mirrors those slots for Python callers.
"""
from . import _abi  # noqa: F401  (raises ImportError when the library is not built)
from ._abi import DeviceBuffer, DevicePanic, VhError, init, sync  # noqa: F401
