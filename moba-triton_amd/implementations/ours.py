"""The MI355X HIP kernels behind the common Backend interface
(reference `implementations/ours.py:32-159`).

Registered as "ours": the same name, methods and availability contract as the
reference's Triton backend, so `bench/suite.py`-style harnesses and the tests
drive it unchanged. Unlike the reference (bf16/fp16 only) this backend also
runs float32, on the library's float32 kernels.
"""

import torch

from implementations.base import register
from moba import _lib
from moba.config import MoBAConfig
from moba.device import TARGET_ARCH, TENSOR_CORE_TILE, device_arch, supports_dtype
from moba.kernels.attention import moba_attention
from moba.kernels.moba_fwd import moba_forward
from moba.kernels.routing import build_csc_fused, csc_to_mask

KERNEL_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


class OursBackend:
    """Adapter for `moba.kernels.moba_fwd.moba_forward` on gfx950."""

    name = "ours"
    vendored = False
    computes_moba = True

    def is_available(self, cfg: MoBAConfig) -> tuple[bool, str]:
        """Never raises (`ours.py:39-80`)."""
        try:
            if not torch.cuda.is_available():
                return False, "no GPU device"
            arch = device_arch(0)
            # The wording of both rejections below is what the reference's
            # registry tests match (tests/test_registry.py:148-164): "tensor-core"
            # for a dtype without a kernel, "tl.dot" for a block below the tile.
            if cfg.dtype not in KERNEL_DTYPES:
                return False, (f"dtype {cfg.dtype} has no tensor-core (MFMA) path; these "
                               "kernels compute in bfloat16, float16 or float32")
            ok, reason = supports_dtype(cfg.dtype, arch.split(":")[0] or TARGET_ARCH)
            if not ok:
                return False, reason
            if cfg.block_size < TENSOR_CORE_TILE:
                return False, (f"block_size {cfg.block_size} is below the MFMA tile minimum "
                               f"(the tl.dot minimum of the Triton reference) of "
                               f"{TENSOR_CORE_TILE}")
            ok, reason = _lib.available()
            if not ok:
                return False, reason
            return True, ""
        except Exception as exc:  # noqa: BLE001 - must never raise
            return False, f"{type(exc).__name__}: {exc}"

    def _require(self, cfg):
        ok, reason = self.is_available(cfg)
        if not ok:
            raise RuntimeError(f"ours backend not available: {reason}")

    def forward_grad(self, q, k, v, cfg: MoBAConfig) -> torch.Tensor:
        """Differentiable forward (`ours.py:82-97`)."""
        self._require(cfg)
        return moba_attention(q, k, v, cfg)

    def forward(self, q, k, v, cfg: MoBAConfig) -> torch.Tensor:
        """Forward only, index rebuilt every call (`ours.py:99-129`).

        Raises:
            RuntimeError: If the backend is unavailable for `cfg`.
            ValueError: If shapes or head_dim are unsupported.
        """
        self._require(cfg)
        return moba_forward(q, k, v, cfg)

    def forward_packed(self, q, k, v, cfg: MoBAConfig, cu_seqlens, max_seqlen=None):
        """Packed ([1, T, H, D]) forward; derives max_seqlen (one host read)
        when it is not given."""
        self._require(cfg)
        if max_seqlen is None:
            max_seqlen = int((cu_seqlens[1:] - cu_seqlens[:-1]).max())
        return moba_forward(q, k, v, cfg, cu_seqlens=cu_seqlens.to(torch.int32),
                            max_seqlen=max_seqlen)

    def selection(self, q, k, cfg: MoBAConfig) -> torch.Tensor:
        """Routing as a dense mask, round-tripped through the CSC index the
        kernels read (`ours.py:131-156`)."""
        self._require(cfg)
        q, k = q.contiguous(), k.contiguous()
        return csc_to_mask(build_csc_fused(q, k, cfg), q.shape[1])


register(OursBackend())
