"""MI355X (gfx950) kernels of the route n-gram memory hot path, behind a C ABI.

``lngram_hip.ops`` holds the tensor-level wrappers; ``lngram_hip.workloads``
the synthetic workload shapes used by the benchmark and the tests.
"""

from . import _lib, ops  # noqa: F401
from ._lib import LibraryMissing, load  # noqa: F401

__all__ = ["ops", "load", "LibraryMissing"]
