"""Backend protocol and registry (reference `implementations/base.py:21-159`).

Every MoBA implementation is reached through one interface so that tests and
benchmarks never special-case one. `is_available` returns a reason string
instead of raising, so a skipped backend can say why.
"""

from typing import Protocol, runtime_checkable

import torch

from moba.config import MoBAConfig


@runtime_checkable
class Backend(Protocol):
    """One MoBA implementation.

    Attributes:
        name: Unique registry key.
        vendored: True for third-party code (compared, never asserted).
        computes_moba: False for a dense baseline.

    Optional methods a backend may add: `forward_grad(q, k, v, cfg)`
    (differentiable), `selection(q, k, cfg) -> bool [B, H, S, nb]`,
    `forward_packed(q, k, v, cfg, cu_seqlens, max_seqlen=None)`.
    """

    name: str
    vendored: bool = False
    computes_moba: bool = True

    def is_available(self, cfg: MoBAConfig) -> tuple[bool, str]:
        """(available, reason); must never raise."""
        ...

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                cfg: MoBAConfig) -> torch.Tensor:
        """MoBA attention, [B, S, H, D] in and out."""
        ...


_REGISTRY: dict[str, Backend] = {}


def register(backend: Backend) -> Backend:
    """Adds a backend; a duplicate name raises ValueError."""
    if backend.name in _REGISTRY:
        raise ValueError(f"Backend {backend.name!r} is already registered")
    _REGISTRY[backend.name] = backend
    return backend


def all_backends() -> list[Backend]:
    """Every registered backend, available or not."""
    return list(_REGISTRY.values())


def get_backend(name: str) -> Backend:
    """Looks up a backend; KeyError lists the registered names."""
    if name not in _REGISTRY:
        raise KeyError(f"No backend named {name!r}; have {sorted(_REGISTRY)}")
    return _REGISTRY[name]


def available_backends(cfg: MoBAConfig) -> list[Backend]:
    """Backends whose `is_available(cfg)` is True."""
    return [b for b in _REGISTRY.values() if b.is_available(cfg)[0]]


def skipped_backends(cfg: MoBAConfig) -> list[tuple[str, str]]:
    """(name, reason) for each backend that cannot run `cfg`."""
    out = []
    for backend in _REGISTRY.values():
        ok, reason = backend.is_available(cfg)
        if not ok:
            out.append((backend.name, reason))
    return out
