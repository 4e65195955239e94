"""chromofold_amd — MI355X-native (gfx950) implementation of chromoFold's decode-in-kernel hot path.

The product is libchromofold.so (HIP kernels + C ABI identical to the reference's include/chromofold headers).
This package is the Python host-side mirror used by tests and benchmarks; it never computes results itself.
"""
from . import _abi  # noqa: F401

__all__ = ["_abi"]
