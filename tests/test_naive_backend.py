"""The naive_torch backend (dense PyTorch MoBA, a comparison baseline) against
the oracle on CPU; mirrors the reference's registry tests that need no GPU
(`tests/test_registry.py:22-73`)."""

import pytest
import torch

from conftest import make_qkv, oracle_cfg
from implementations import all_backends, available_backends, get_backend, skipped_backends
from moba.config import MoBAConfig
from oracle import naive as O


def test_naive_torch_is_always_available():
    ok, reason = get_backend("naive_torch").is_available(MoBAConfig(block_size=32, top_k=2))
    assert ok, reason


def test_available_and_skipped_partition_the_registry():
    cfg = MoBAConfig(block_size=32, top_k=2)
    assert len(available_backends(cfg)) + len(skipped_backends(cfg)) == len(all_backends())
    for name, reason in skipped_backends(cfg):
        assert reason, name


def test_is_available_never_raises_on_absurd_config():
    cfg = MoBAConfig(block_size=1, top_k=999999, dtype=torch.float64)
    for backend in all_backends():
        ok, reason = backend.is_available(cfg)
        assert isinstance(ok, bool) and isinstance(reason, str)


def test_unknown_backend_lists_naive_torch():
    with pytest.raises(KeyError, match="naive_torch"):
        get_backend("does_not_exist")


@pytest.mark.parametrize("shape,h_kv,bs,tk", [((1, 512, 4, 64), 4, 32, 4),
                                              ((2, 300, 4, 32), 2, 64, 3),
                                              ((1, 256, 2, 64), 1, 16, 8)])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_naive_torch_matches_the_oracle(shape, h_kv, bs, tk, dtype):
    cfg = MoBAConfig(block_size=bs, top_k=tk, dtype=dtype)
    q, k, v = make_qkv(shape, dtype, seed=11)
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    backend = get_backend("naive_torch")
    sel = O.moba_selection(q, k, oracle_cfg(cfg))
    assert torch.equal(backend.selection(q, k, cfg), sel)
    want = O.moba_attention(q, k, v, oracle_cfg(cfg), selected=sel)
    got = backend.forward(q, k, v, cfg)
    assert got.dtype is dtype and got.shape == q.shape
    tol = 1e-10 if dtype == torch.float64 else 2e-6
    torch.testing.assert_close(got, want, rtol=tol, atol=tol)


def test_naive_torch_bf16_selection_matches_the_oracle():
    cfg = MoBAConfig(block_size=32, top_k=4)
    q, k, _ = make_qkv((1, 1024, 2, 64), torch.bfloat16, seed=3)
    sel = O.moba_selection(q, k, oracle_cfg(cfg))
    assert torch.equal(get_backend("naive_torch").selection(q, k, cfg), sel)


def test_naive_torch_reduces_to_dense_when_every_block_is_selected():
    b, s, h, d = 1, 64, 2, 32
    q, k, v = make_qkv((b, s, h, d), torch.float64, seed=0)
    cfg = MoBAConfig(block_size=16, top_k=s // 16, dtype=torch.float64)
    got = get_backend("naive_torch").forward(q, k, v, cfg)
    want = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True).transpose(1, 2)
    torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-10)


def test_naive_torch_packed_equals_each_sequence_alone():
    cfg = MoBAConfig(block_size=16, top_k=3, dtype=torch.float64)
    cu = torch.tensor([0, 80, 128, 200], dtype=torch.int32)
    q, k, v = make_qkv((1, 200, 2, 32), torch.float64, seed=5)
    backend = get_backend("naive_torch")
    packed = backend.forward_packed(q, k, v, cfg, cu)
    sel = O.moba_selection(q, k, oracle_cfg(cfg), cu_seqlens=cu)
    want = O.moba_attention(q, k, v, oracle_cfg(cfg), selected=sel, cu_seqlens=cu)
    torch.testing.assert_close(packed, want, rtol=1e-10, atol=1e-10)


def test_naive_torch_gradients_match_the_oracle():
    cfg = MoBAConfig(block_size=16, top_k=3, dtype=torch.float64)
    q, k, v = make_qkv((1, 128, 2, 32), torch.float64, seed=9)
    do = torch.randn_like(q)
    a = [t.clone().requires_grad_(True) for t in (q, k, v)]
    get_backend("naive_torch").forward_grad(*a, cfg).backward(do)
    bref = [t.clone().requires_grad_(True) for t in (q, k, v)]
    sel = O.moba_selection(q, k, oracle_cfg(cfg))
    O.moba_attention(*bref, oracle_cfg(cfg), selected=sel).backward(do)
    for x, y in zip(a, bref):
        torch.testing.assert_close(x.grad, y.grad, rtol=1e-9, atol=1e-9)


def test_naive_torch_packed_is_differentiable():
    """Packed gradients equal those of the oracle's packed attention."""
    cfg = MoBAConfig(block_size=16, top_k=3, dtype=torch.float64)
    cu = torch.tensor([0, 80, 128, 200], dtype=torch.int32)
    q, k, v = make_qkv((1, 200, 2, 32), torch.float64, seed=6)
    do = torch.randn_like(q)
    a = [t.clone().requires_grad_(True) for t in (q, k, v)]
    get_backend("naive_torch").forward_packed(*a, cfg, cu).backward(do)
    bref = [t.clone().requires_grad_(True) for t in (q, k, v)]
    sel = O.moba_selection(q, k, oracle_cfg(cfg), cu_seqlens=cu)
    O.moba_attention(*bref, oracle_cfg(cfg), selected=sel, cu_seqlens=cu).backward(do)
    for x, y in zip(a, bref):
        torch.testing.assert_close(x.grad, y.grad, rtol=1e-9, atol=1e-9)
