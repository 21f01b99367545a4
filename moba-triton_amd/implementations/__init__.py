"""Backend registry; importing registers the built-in backends
(reference `implementations/__init__.py:20-32`).

Built in: "ours" (the HIP kernels), "naive_torch" (dense PyTorch MoBA, a
comparison baseline on any device) and "sdpa_dense" (torch's dense causal
SDPA, the baseline of the attainment figure; not MoBA). The packed varlen
signature `moba_attn_varlen_triton` is in `implementations.triton_moba` and
is not a registered backend.
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
from implementations import naive_torch as _naive_torch  # noqa: F401
from implementations import sdpa_dense as _sdpa_dense  # noqa: F401

__all__ = ["Backend", "all_backends", "available_backends", "get_backend", "register",
           "skipped_backends"]
