"""Packed-batch metadata checks (`src/moba/varlen.py:33-111`).

`validate_cu_seqlens` runs on every call, so value checks happen only when
`cu_seqlens` lives on the CPU (or `strict=True`): on a device tensor they
would each cost a host synchronisation.
"""

import torch


def validate_cu_seqlens(cu_seqlens: torch.Tensor, total_tokens: int,
                        max_seqlen: int, strict: bool = False) -> int:
    """Checks packed metadata and returns the sequence count.

    Structural checks (rank, length, int32 dtype, positive max_seqlen)
    always run; value checks (starts at 0, strictly increasing, ends at
    `total_tokens`, no sequence above `max_seqlen`) run on CPU tensors or
    with `strict`.

    Raises:
        ValueError: On any failed check.
    """
    if cu_seqlens.ndim != 1:
        raise ValueError(f"cu_seqlens must be 1-D, got shape {tuple(cu_seqlens.shape)}")
    if cu_seqlens.numel() < 2:
        raise ValueError(
            f"cu_seqlens needs at least two entries (one sequence), got "
            f"{cu_seqlens.numel()}")
    if cu_seqlens.dtype != torch.int32:
        raise ValueError(f"cu_seqlens must be int32, got {cu_seqlens.dtype}")
    if max_seqlen <= 0:
        raise ValueError(f"max_seqlen must be positive, got {max_seqlen}")
    n = cu_seqlens.numel() - 1
    if cu_seqlens.device.type == "cpu" or strict:
        cu = cu_seqlens.cpu()
        if int(cu[0]) != 0:
            raise ValueError(f"cu_seqlens must start at 0, got {int(cu[0])}")
        lengths = cu[1:] - cu[:-1]
        if bool((lengths <= 0).any()):
            raise ValueError(
                f"cu_seqlens must be strictly increasing (no empty sequence), "
                f"got lengths {lengths.tolist()}")
        if int(cu[-1]) != total_tokens:
            raise ValueError(
                f"cu_seqlens ends at {int(cu[-1])} but the total token count is "
                f"{total_tokens}")
        longest = int(lengths.max())
        if longest > max_seqlen:
            raise ValueError(
                f"max_seqlen {max_seqlen} is below the longest sequence {longest}")
    return n
