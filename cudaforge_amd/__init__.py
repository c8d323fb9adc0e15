"""cudaforge_amd — MI355X (gfx950) attention hot path behind CudaForge's operator API.

The product is the C-ABI shared library ``libcudaforge_amd.so`` in this directory
(declared by ``include/*.h``).  This package only loads it and offers thin ctypes
helpers (device buffers, params structs, operator calls) for tests and the benchmark.
There is no CPU fallback: if the library is missing, importing the helpers raises.
"""

from ._native import LIB_PATH, NativeLibraryMissing, lib, load_library  # noqa: F401
from .api import (  # noqa: F401
    DeviceBuffer,
    MhaDecodeParams,
    MhaFusedParams,
    MhaDecodeRopeParams,
    RopeParams,
    LayerNormParams,
    MatmulParams,
    CastParams,
    CausalMaskParams,
    GraphMhaMatch,
    OperatorRegistry,
    Stream,
    Event,
    TensorT,
    call_entry,
    call_op,
    device_caps,
    find_op,
    graph_detect_mha,
    gpu_available,
    init_gpu,
)
