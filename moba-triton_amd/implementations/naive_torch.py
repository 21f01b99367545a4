"""Dense PyTorch MoBA as a backend (reference `implementations/naive_torch.py:10-56`).

The slow, obvious form of the same function: an [S, S] score matrix per
head, masked to each query's selected blocks, on whatever device the inputs
live on (CPU included). It is a comparison baseline for harnesses that list
every backend; the product path is the "ours" backend, which runs the HIP
library and never falls back to this.

Semantics (reference `src/moba/naive.py:23-146, 224-330`):
  - block representative = block mean over the keys the block holds, the sum
    taken in float32 and rounded to the dtype, then divided in the dtype;
  - gate score = q . kbar accumulated in float32, rounded to the dtype;
  - a query selects its own block plus the `past_blocks_selected` best
    strictly-past blocks, ranked by (score desc, block id asc);
  - softmax over the selected keys with the causal mask, in float32 (float64
    for float64 inputs).
"""

import math

import torch

from implementations.base import register
from moba.config import MoBAConfig
from moba.gqa import head_group_size


def _block_means(k: torch.Tensor, block_size: int) -> torch.Tensor:
    """[B, S, H, D] -> [B, H, nb, D] block means, short tail by its count."""
    b, s, h, d = k.shape
    nb = math.ceil(s / block_size)
    block_of = torch.arange(s, device=k.device) // block_size
    sums = torch.zeros(b, nb, h, d, device=k.device, dtype=torch.float32)
    sums.index_add_(1, block_of, k.float())
    occupancy = torch.bincount(block_of, minlength=nb).to(k.dtype)
    return (sums.to(k.dtype) / occupancy.view(1, nb, 1, 1)).transpose(1, 2)


def _selection(q: torch.Tensor, k: torch.Tensor, cfg: MoBAConfig) -> torch.Tensor:
    """bool [B, H, S, nb]: which blocks each query attends."""
    b, s, h, _ = q.shape
    group = head_group_size(h, k.shape[2])
    kbar = _block_means(k, cfg.block_size)
    if group > 1:
        kbar = kbar.repeat_interleave(group, dim=1)
    nb = kbar.shape[2]
    score = torch.matmul(q.float().transpose(1, 2), kbar.float().transpose(-1, -2))
    score = score.to(q.dtype)
    own = (torch.arange(s, device=q.device) // cfg.block_size).view(s, 1)
    ids = torch.arange(nb, device=q.device).view(1, nb)
    past = ids < own
    take = cfg.past_blocks_selected(nb)
    ranked = score.float().masked_fill(~past, -math.inf)
    # Stable descending sort: equal scores keep ascending block order.
    order = torch.sort(ranked, dim=-1, descending=True, stable=True).indices[..., :take]
    chosen = torch.zeros(b, h, s, nb, dtype=torch.bool, device=q.device)
    chosen.scatter_(-1, order, True)
    chosen &= past
    if cfg.always_select_current:
        chosen |= ids == own
    return chosen


def _attend(q, k, v, sel, block_size):
    """Dense masked softmax attention over the selected blocks."""
    b, s, h, d = q.shape
    group = head_group_size(h, k.shape[2])
    ct = torch.promote_types(q.dtype, torch.float32)
    kh, vh = (t.transpose(1, 2).to(ct) for t in (k, v))
    if group > 1:
        kh, vh = (t.repeat_interleave(group, dim=1) for t in (kh, vh))
    logits = torch.matmul(q.transpose(1, 2).to(ct), kh.transpose(-1, -2)) / math.sqrt(d)
    key_block = torch.arange(s, device=q.device) // block_size
    allowed = sel[..., key_block]
    allowed &= torch.ones(s, s, dtype=torch.bool, device=q.device).tril()
    logits = logits.masked_fill(~allowed, -math.inf)
    out = torch.matmul(torch.softmax(logits, dim=-1), vh)
    return out.transpose(1, 2).to(q.dtype)


class NaiveTorchBackend:
    """Pure-PyTorch MoBA; available wherever torch runs."""

    name = "naive_torch"
    vendored = False
    computes_moba = True

    def is_available(self, cfg: MoBAConfig) -> tuple[bool, str]:
        return True, ""

    def forward(self, q, k, v, cfg: MoBAConfig) -> torch.Tensor:
        with torch.no_grad():
            return self.forward_grad(q, k, v, cfg)

    def forward_grad(self, q, k, v, cfg: MoBAConfig) -> torch.Tensor:
        """Differentiable (plain autograd through the dense form)."""
        if k.shape != v.shape or q.shape[:2] != k.shape[:2] or q.shape[-1] != k.shape[-1]:
            raise ValueError(f"incompatible shapes q {tuple(q.shape)}, k {tuple(k.shape)}, "
                             f"v {tuple(v.shape)}")
        sel = _selection(q.detach(), k.detach(), cfg)
        return _attend(q, k, v, sel, cfg.block_size)

    def forward_packed(self, q, k, v, cfg: MoBAConfig, cu_seqlens, max_seqlen=None):
        """[1, T, H, D] packed: every sequence on its own, sequence-local
        blocks. Differentiable like `forward_grad` (the pieces are joined with
        torch.cat, so gradients reach q, k and v of every sequence)."""
        if q.shape[0] != 1:
            raise ValueError(f"packed input must have batch 1, got {q.shape[0]}")
        bounds = [int(x) for x in cu_seqlens.tolist()]
        pieces = [self.forward_grad(q[:, lo:hi], k[:, lo:hi], v[:, lo:hi], cfg)
                  for lo, hi in zip(bounds[:-1], bounds[1:]) if hi > lo]
        if not pieces:
            return torch.empty_like(q)
        return torch.cat(pieces, dim=1)

    def selection(self, q, k, cfg: MoBAConfig) -> torch.Tensor:
        """bool [B, H, S, nb]."""
        return _selection(q, k, cfg)


register(NaiveTorchBackend())
