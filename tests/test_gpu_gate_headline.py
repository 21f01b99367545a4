"""The gate at the headline size, [1, 524288, 4, 64] (4096 blocks of 128),
against the C oracle on whole heads, on the three key distributions the
bench times: i.i.d. N(0, 1) keys, a random walk along the sequence plus unit
noise, and a per-channel offset shared by every token plus unit noise (the
trained-key case, whose block representatives nearly coincide so that many
scores round to the same key).

Per case: every query of head 0 and every eighth query (a different phase
per head, so every 128-query workgroup is covered) of the other heads are
compared with `oracle.c_oracle.gate_select_strided` (semantics
src/moba/naive.py:64-146), exactly. The gate's workspace counters say which
decision path ran: offset keys must send queries to the fallback kernel
(the settle/fallback logic depends on the block count, and this is its
heaviest regime), whose (key, id)-ordered lists settle the ties; what it
cannot settle goes on to the exact queue kernel.
"""

import pytest
import torch

from conftest import oracle_cfg
from moba import _lib
from moba.config import MoBAConfig
from moba.kernels.pooling import pool_blocks
from oracle import c_oracle

pytestmark = pytest.mark.gpu

S, H, D, BS = 524288, 4, 64, 128


def _keys(kind, dtype, dev):
    """The bench's inputs (`bench.py:hierarchical_gate`): q, then the i.i.d.,
    walk and offset keys, in that order from one seeded device generator."""
    g = torch.Generator(device=dev).manual_seed(1)
    shape = (1, S, H, D)
    q = torch.randn(shape, generator=g, device=dev, dtype=torch.bfloat16)
    k = torch.randn(shape, generator=g, device=dev, dtype=torch.bfloat16)
    if kind != "iid":
        walk = torch.randn(shape, generator=g, device=dev).mul_(0.05).cumsum_(1)
        k = (walk + torch.randn(shape, generator=g, device=dev)).to(torch.bfloat16)
        del walk
    if kind == "offset":
        k = (3.0 * torch.randn((1, 1, H, D), generator=g, device=dev)
             + torch.randn(shape, generator=g, device=dev)).to(torch.bfloat16)
    return q.to(dtype), k.to(dtype)


def _gate_with_counters(q, kbar, cfg):
    b, s, h, d = q.shape
    n = kbar.shape[2]
    ws = torch.zeros(int(_lib.load().moba_gate_workspace_size(b, s, h)), dtype=torch.uint8,
                     device=q.device)
    out = torch.full((b, h, s, cfg.slots()), -7, dtype=torch.int32, device=q.device)
    _lib.call("moba_gate", _lib.ptr(q), _lib.ptr(kbar), _lib.ptr(out), None, b, s, s, h,
              kbar.shape[1], d, n, cfg.block_size, cfg.slots(), cfg.past_blocks_selected(n),
              int(bool(cfg.always_select_current)), _lib.DTYPE_CODE[q.dtype], _lib.ptr(ws),
              ws.numel(), _lib.stream_handle(q.device))
    torch.cuda.synchronize()
    queued, fallback = ws[:8].view(torch.int32).tolist()
    return out.cpu(), queued, fallback


def _compare(got, want, label):
    bad = (got != want).any(-1)
    assert not bool(bad.any()), (
        f"{label}: {int(bad.sum())} of {bad.numel()} queries route differently; first "
        f"{torch.nonzero(bad)[0].tolist()}: got {got[bad][0].tolist()} "
        f"want {want[bad][0].tolist()}")


@pytest.mark.parametrize("kind,dtype,top_k", [
    ("iid", torch.bfloat16, 8),
    ("walk", torch.bfloat16, 8),
    ("offset", torch.bfloat16, 8),
    ("offset", torch.float16, 8),
    ("offset", torch.bfloat16, 16),
])
def test_gate_headline_whole_heads_match_oracle(device, kind, dtype, top_k):
    cfg = MoBAConfig(block_size=BS, top_k=top_k, dtype=dtype)
    q, k = _keys(kind, dtype, device)
    kbar = pool_blocks(k, cfg)
    del k
    got, queued, fallback = _gate_with_counters(q, kbar, cfg)
    print(f"[gate-512k] {kind} {dtype} top_k={top_k}: queued {queued}, "
          f"fallback tiles {fallback}", flush=True)
    qc, kc = q.cpu(), kbar.cpu()
    del q, kbar
    ocfg = oracle_cfg(cfg)
    want0 = c_oracle.gate_select_strided(qc, kc, ocfg, heads=range(0, 1))
    _compare(got[:, 0:1], want0, f"{kind} head 0 (all {S} queries)")
    for h in range(1, H):
        off = (3 * h) % 8
        want = c_oracle.gate_select_strided(qc, kc, ocfg, heads=range(h, h + 1), offset=off,
                                            stride=8)
        _compare(got[:, h:h + 1, off::8], want, f"{kind} head {h} (every 8th from {off})")
    if kind == "offset":
        # The regime this test exists for: near-tied boundary keys that the
        # one-stream decision cannot settle.
        assert fallback > 0, "offset keys did not reach the fallback kernel"
