"""Dense causal attention baseline (reference `implementations/sdpa_dense.py:1-120`).

Not MoBA: torch's `scaled_dot_product_attention` over every causally legal
key, the anchor of the attainment figure (speedup over dense divided by the
speedup the sparsity pattern makes available, reference `bench/suite.py:1-12,
549-583`). Only the fused SDPA kernels are allowed: the math path would
materialise an S x S score matrix, which at the benchmark lengths does not
fit; it is allowed only up to MATH_MAX_SEQ tokens (small test shapes in
dtypes without a fused kernel), and past that a shape with no fused kernel
raises.
"""

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from implementations.base import register
from moba.config import MoBAConfig
from moba.gqa import head_group_size

FUSED = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]
MATH_MAX_SEQ = 8192


class SdpaDenseBackend:
    """torch SDPA, causal, dense, on the current GPU."""

    name = "sdpa_dense"
    vendored = False
    computes_moba = False

    def is_available(self, cfg: MoBAConfig) -> tuple[bool, str]:
        """Never raises."""
        try:
            if not torch.cuda.is_available():
                return False, "no GPU device"
            return True, ""
        except Exception as exc:  # noqa: BLE001 - must never raise
            return False, f"availability probe failed: {exc}"

    @staticmethod
    def _dense(q, k, v):
        # SDPA is head-major; grouped kv heads are repeated to the query heads.
        group = head_group_size(q.shape[2], k.shape[2])
        if group > 1:
            k, v = (t.repeat_interleave(group, dim=2) for t in (k, v))
        qh, kh, vh = (t.transpose(1, 2) for t in (q, k, v))
        # The math path materialises S x S scores: allowed only where that is
        # small (dtypes without a fused kernel, e.g. float64, at test sizes).
        allowed = FUSED + ([SDPBackend.MATH] if q.shape[1] <= MATH_MAX_SEQ else [])
        with sdpa_kernel(allowed):
            out = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True)
        return out.transpose(1, 2)

    def forward(self, q, k, v, cfg: MoBAConfig) -> torch.Tensor:
        """Ignores the gate parameters by design: attends to everything."""
        with torch.no_grad():
            return self._dense(q, k, v)

    def forward_grad(self, q, k, v, cfg: MoBAConfig) -> torch.Tensor:
        """Differentiable form of `forward`."""
        return self._dense(q, k, v)

    def forward_packed(self, q, k, v, cfg: MoBAConfig, cu_seqlens) -> torch.Tensor:
        """Dense causal attention per packed sequence ([1, T, H, D] with
        `cu_seqlens`), one SDPA call each, so no padding is attended."""
        bounds = cu_seqlens.tolist()
        out = torch.empty_like(q)
        with torch.no_grad():
            for lo, hi in zip(bounds[:-1], bounds[1:]):
                if hi > lo:
                    out[:, lo:hi] = self._dense(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi])
        return out


register(SdpaDenseBackend())
