"""Backend registry; importing registers the built-in backends
(reference `implementations/__init__.py:20-32`).

Built in: "ours" (the HIP kernels) and "triton_moba" (the same kernels
behind the packed varlen signature).
"""

from implementations.base import (
    Backend,
    all_backends,
    available_backends,
    get_backend,
    register,
    skipped_backends,
)
from implementations import ours as _ours  # noqa: F401
from implementations import triton_moba as _triton_moba  # noqa: F401

__all__ = ["Backend", "all_backends", "available_backends", "get_backend", "register",
           "skipped_backends"]
