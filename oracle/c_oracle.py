"""ctypes front end of `moba_oracle.c` (test infrastructure only).

Same semantics as `oracle.naive.pool_blocks` / `gate_select`, streaming, so
it reaches S = 64K+ without a dense score matrix. Inputs are CPU tensors.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import torch

from oracle.naive import num_blocks, past_blocks_selected, slots_per_query

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libmoba_oracle.so"
_lib = None

_DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def build() -> Path:
    """Compiles the C oracle with its Makefile (gcc only, no reference code)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        P, I = ctypes.c_void_p, ctypes.c_int
        _lib.oracle_pool.argtypes = [P, I, I, I, I, I, I, P, I, I, P]
        _lib.oracle_gate.argtypes = [P, P, I, I, I, I, I, I, I, I, I, I, I,
                                     P, I, P]
        _lib.oracle_gate_strided.argtypes = [P, P] + [I] * 15 + [P]
    return _lib


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def pool_blocks(k: torch.Tensor, block_size: int, cu_seqlens=None,
                max_seqlen=None) -> torch.Tensor:
    """`[B, S, H, D]` -> `[B or n_seq, H, nb, D]` in k.dtype."""
    b, s, h, d = k.shape
    kf = k.detach().cpu().to(torch.float32).contiguous()
    if cu_seqlens is None:
        n = num_blocks(s, block_size)
        rows, cu, n_seq = b, None, 0
    else:
        n = num_blocks(int(max_seqlen), block_size)
        cu = cu_seqlens.cpu().to(torch.int32).contiguous()
        n_seq = cu.numel() - 1
        rows = n_seq
    out = torch.zeros(rows, h, n, d, dtype=torch.float32)
    lib().oracle_pool(_ptr(kf), b, s, h, d, block_size, _DTYPE_CODE[k.dtype],
                      _ptr(cu) if cu is not None else None, n_seq, n,
                      _ptr(out))
    return out.to(k.dtype)


def gate_select(q: torch.Tensor, kbar: torch.Tensor, cfg, cu_seqlens=None,
                max_seqlen=None) -> torch.Tensor:
    """Selected ids `[B, Hq, S, slots]` int32, ascending, -1 padded."""
    b, s, hq, d = q.shape
    hkv, n = kbar.shape[1], kbar.shape[2]
    qf = q.detach().cpu().to(torch.float32).contiguous()
    kf = kbar.detach().cpu().to(torch.float32).contiguous()
    slots = slots_per_query(cfg)
    if cu_seqlens is None:
        take = past_blocks_selected(cfg, n)
        cu, n_seq = None, 0
    else:
        take = past_blocks_selected(cfg, num_blocks(int(max_seqlen),
                                                    cfg.block_size))
        cu = cu_seqlens.cpu().to(torch.int32).contiguous()
        n_seq = cu.numel() - 1
    out = torch.empty(b, hq, s, slots, dtype=torch.int32)
    lib().oracle_gate(_ptr(qf), _ptr(kf), b, s, hq, hkv, d, n,
                      cfg.block_size, take, int(bool(cfg.always_select_current)),
                      slots, _DTYPE_CODE[q.dtype],
                      _ptr(cu) if cu is not None else None, n_seq, _ptr(out))
    return out


def gate_select_strided(q: torch.Tensor, kbar: torch.Tensor, cfg, heads=None,
                        offset: int = 0, stride: int = 1) -> torch.Tensor:
    """`gate_select` of a padded batch restricted to query heads `heads`
    (a range; all by default) and rows offset, offset + stride, ...:
    ids `[B, len(heads), ceil((S - offset) / stride), slots]` int32."""
    b, s, hq, d = q.shape
    hkv, n = kbar.shape[1], kbar.shape[2]
    heads = range(hq) if heads is None else heads
    assert heads.step == 1 and 0 <= heads.start < heads.stop <= hq
    qf = q.detach().cpu().to(torch.float32).contiguous()
    kf = kbar.detach().cpu().to(torch.float32).contiguous()
    slots = slots_per_query(cfg)
    nt = max(0, -(-(s - offset) // stride))
    out = torch.empty(b, len(heads), nt, slots, dtype=torch.int32)
    lib().oracle_gate_strided(_ptr(qf), _ptr(kf), b, s, hq, hkv, d, n, cfg.block_size,
                              past_blocks_selected(cfg, n),
                              int(bool(cfg.always_select_current)), slots,
                              _DTYPE_CODE[q.dtype], heads.start, heads.stop, offset, stride,
                              _ptr(out))
    return out


def set_threads(n: int) -> None:
    os.environ["OMP_NUM_THREADS"] = str(n)
