"""The opt-in hierarchical gate (cfg.gate_group > 0) on the GPU against the
oracle's `hierarchical_select`: ids bit-exact, the identities that reduce it
to the exact gate, and its use inside attention."""

import pytest
import torch

from conftest import make_qkv, oracle_cfg
from moba.config import MoBAConfig
from moba.kernels.gating import gate_select
from moba.kernels.pooling import pool_blocks
from oracle import c_oracle
from oracle import naive as O

pytestmark = pytest.mark.gpu


def _check(q, k, cfg, rows=None):
    kbar = pool_blocks(k, cfg)
    got = gate_select(q, kbar, cfg).cpu()
    kb = kbar.cpu()
    sel = O.hierarchical_select(q.cpu(), kb, oracle_cfg(cfg), cfg.gate_group, cfg.gate_open,
                                rows=rows)
    want = O.mask_to_indices(sel, cfg.slots())
    if rows is not None:
        got = got[:, :, rows]
    bad = (got != want).any(-1)
    assert not bool(bad.any()), (
        f"{int(bad.sum())} queries differ; first {torch.nonzero(bad)[0].tolist()}: "
        f"got {got[bad][0].tolist()} want {want[bad][0].tolist()}")
    return got


@pytest.mark.parametrize("shape,h_kv,bs,tk,group,opened", [
    ((1, 4096, 4, 64), 4, 32, 8, 8, 4),
    ((2, 2048, 4, 64), 2, 64, 5, 4, 3),
    ((1, 4096, 8, 128), 2, 32, 8, 16, 6),
    ((1, 3000, 2, 64), 2, 16, 4, 32, 2),
    ((1, 8192, 4, 64), 4, 128, 8, 4, 8),
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_hierarchical_gate_matches_oracle(device, shape, h_kv, bs, tk, group, opened, dtype):
    cfg = MoBAConfig(block_size=bs, top_k=tk, dtype=dtype, gate_group=group, gate_open=opened)
    q, k, _ = make_qkv(shape, dtype, seed=17, device=device)
    _check(q, k[:, :, :h_kv].contiguous(), cfg)


def test_hierarchical_gate_opening_everything_is_the_exact_gate(device):
    shape = (1, 32768, 4, 64)
    q, k, _ = make_qkv(shape, torch.bfloat16, seed=18, device=device)
    exact = gate_select(q, pool_blocks(k, MoBAConfig(128, 8)), MoBAConfig(128, 8))
    # 256 blocks in super-blocks of 4: 64 super-blocks, all opened.
    cfg = MoBAConfig(128, 8, gate_group=4, gate_open=64)
    assert torch.equal(gate_select(q, pool_blocks(k, cfg), cfg), exact)
    # Super-blocks of one block, as many opened as the past budget.
    cfg = MoBAConfig(128, 8, gate_group=1, gate_open=7)
    assert torch.equal(gate_select(q, pool_blocks(k, cfg), cfg), exact)


def test_hierarchical_gate_sampled_rows_at_the_headline_size(device):
    cfg = MoBAConfig(128, 8, gate_group=16, gate_open=8)
    q, k, _ = make_qkv((1, 524288, 4, 64), torch.bfloat16, seed=0, device=device)
    rows = torch.tensor(sorted({0, 127, 128, 2047, 2048, 65535, 131072, 300001, 524287} |
                               set(range(5, 524288, 21011))))
    _check(q, k, cfg, rows=rows)


def test_hierarchical_gate_in_attention_and_packed_rejected(device):
    from moba.kernels.attention import moba_attention
    from moba.kernels.routing import build_csc_fused, csc_to_mask

    cfg = MoBAConfig(64, 4, gate_group=4, gate_open=2)
    q, k, v = make_qkv((1, 2048, 2, 64), torch.bfloat16, seed=19, device=device)
    index = build_csc_fused(q, k, cfg)
    sel = O.hierarchical_select(q.cpu(), O.pool_blocks(k.cpu(), 64), oracle_cfg(cfg), 4, 2)
    assert torch.equal(csc_to_mask(index, 2048).cpu(), sel)
    out = moba_attention(q, k, v, cfg)
    ref = O.moba_attention(q.cpu().double(), k.cpu().double(), v.cpu().double(),
                           oracle_cfg(cfg), selected=sel)
    assert (out.cpu().double() - ref).abs().max().item() <= 2e-2
    cu = torch.tensor([0, 1024, 2048], dtype=torch.int32, device=device)
    with pytest.raises(ValueError, match="padded input only"):
        moba_attention(q, k, v, cfg, cu_seqlens=cu, max_seqlen=1024)


def test_refine_ignores_super_block_ids_that_hold_no_block(device):
    """Ids past the last super-block (here large enough that id * group
    overflows int32) and negative ids other than -1 select nothing: each
    query keeps only its own block."""
    from moba import _lib

    b, s, h, d, bs, group = 1, 1024, 2, 64, 64, 4
    q, k, _ = make_qkv((b, s, h, d), torch.bfloat16, seed=33, device=device)
    kbar = pool_blocks(k, MoBAConfig(bs, 4))
    sup = torch.tensor([1 << 30, -5, 4], dtype=torch.int32, device=device).expand(b, h, s, 3)
    sup = sup.contiguous()
    out = torch.full((b, h, s, 4), -7, dtype=torch.int32, device=device)
    _lib.call("moba_gate_refine", _lib.ptr(q), _lib.ptr(kbar), _lib.ptr(sup), _lib.ptr(out), b, s,
              h, h, d, s // bs, bs, group, 3, 4, 3, 1, _lib.DTYPE_CODE[q.dtype],
              _lib.stream_handle(device))
    got = out.cpu()
    own = (torch.arange(s) // bs).view(1, 1, s).expand(b, h, s)
    assert torch.equal(got[..., 0], own)
    assert bool((got[..., 1:] == -1).all())
