"""Backend registry; importing registers the built-in backends
(reference `implementations/__init__.py:20-32`).

Built in: "ours" (the HIP kernels), "triton_moba" (the same kernels behind
the packed varlen signature) and "sdpa_dense" (torch's dense causal SDPA,
the baseline of the attainment figure; not MoBA).
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
from implementations import sdpa_dense as _sdpa_dense  # noqa: F401

__all__ = ["Backend", "all_backends", "available_backends", "get_backend", "register",
           "skipped_backends"]
