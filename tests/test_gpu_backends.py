"""The drop-in surface on the GPU: the registered backends and the packed
varlen signature, against the oracle. Mirrors the reference's
`tests/test_registry.py:75-180` and `tests/test_backends.py:39-127`."""

import pytest
import torch

from conftest import make_qkv, oracle_cfg, sweep_cases
from gpu_util import fp64_truth, oracle_selection, to_cpu
from implementations import available_backends, get_backend
from implementations.triton_moba import moba_attn_varlen_triton
from moba.config import MoBAConfig
from oracle import naive as O
from tolerance import (BF16_MAX_ABS, BF16_MEAN_ABS, assert_selection_matches,
                       assert_within_tolerance, max_abs_error, mean_abs_error)

pytestmark = pytest.mark.gpu


def test_ours_is_registered_available_and_first_party(device):
    backend = get_backend("ours")
    ok, reason = backend.is_available(MoBAConfig(block_size=32, top_k=2, dtype=torch.bfloat16))
    assert ok, reason
    assert backend.vendored is False
    assert callable(getattr(backend, "selection", None))


def test_ours_declines_dtypes_without_a_tensor_core_path(device):
    ok, reason = get_backend("ours").is_available(
        MoBAConfig(block_size=32, top_k=2, dtype=torch.float64))
    assert not ok
    assert "tensor-core" in reason, reason


def test_ours_declines_block_sizes_below_the_tile(device):
    ok, reason = get_backend("ours").is_available(
        MoBAConfig(block_size=8, top_k=2, dtype=torch.bfloat16))
    assert not ok
    assert "tl.dot" in reason, reason


def test_ours_routing_matches_the_oracle(device):
    cfg = MoBAConfig(block_size=32, top_k=2, dtype=torch.bfloat16)
    q, k = make_qkv((1, 256, 2, 64), torch.bfloat16, seed=0, device=device, n=2)
    got = get_backend("ours").selection(q, k, cfg)
    assert got.dtype is torch.bool and got.device.type == "cuda"
    assert torch.equal(got.cpu(), oracle_selection(q, k, cfg))


def test_naive_and_sdpa_agree_when_top_k_covers_all_blocks(device):
    b, h, s, d = 1, 2, 64, 32
    q, k, v = make_qkv((b, s, h, d), torch.float64, seed=0, device=device)
    cfg = MoBAConfig(block_size=16, top_k=s // 16, dtype=torch.float64)
    got = get_backend("naive_torch").forward(q, k, v, cfg)
    want = get_backend("sdpa_dense").forward(q, k, v, cfg)
    torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-10)


def test_backends_preserve_shape_and_dtype(device):
    b, s, h, d = 1, 64, 2, 64
    cfg = MoBAConfig(block_size=16, top_k=2, dtype=torch.bfloat16)
    q, k, v = make_qkv((b, s, h, d), torch.bfloat16, seed=1, device=device)
    names = []
    for backend in available_backends(cfg):
        out = backend.forward(q, k, v, cfg)
        assert out.shape == (b, s, h, d), backend.name
        assert out.dtype is torch.bfloat16, backend.name
        names.append(backend.name)
    assert "ours" in names


def _fast_cases():
    return [c for c in sweep_cases(include_long=False)]


@pytest.mark.parametrize("shape,gate", _fast_cases())
def test_backend_matches_oracle(device, shape, gate):
    """Every first-party MoBA backend's forward within the tolerance policy,
    routing held fixed (reference tests/test_backends.py:39-77)."""
    b, s, h, d = shape
    cfg = MoBAConfig(block_size=gate[0], top_k=gate[1], dtype=torch.bfloat16)
    q, k, v = make_qkv(shape, torch.bfloat16, device=device)
    sel = oracle_selection(q, k, cfg)
    truth, ref_err = fp64_truth(q, k, v, cfg, sel)
    checked = []
    for backend in available_backends(cfg):
        if not backend.computes_moba:
            continue
        out = backend.forward(q, k, v, cfg)
        assert out.shape == (b, s, h, d), backend.name
        assert out.dtype is cfg.dtype, backend.name
        assert bool(torch.isfinite(out).all()), backend.name
        if backend.vendored:
            continue
        assert_within_tolerance(out, truth, ref_err, backend.name)
        checked.append(backend.name)
    assert "ours" in checked


@pytest.mark.parametrize("shape,gate", _fast_cases())
def test_backend_routing_matches_oracle(device, shape, gate):
    cfg = MoBAConfig(block_size=gate[0], top_k=gate[1], dtype=torch.bfloat16)
    q, k, _ = make_qkv(shape, torch.bfloat16, device=device)
    expected = oracle_selection(q, k, cfg)
    exercised = 0
    for backend in available_backends(cfg):
        routing = getattr(backend, "selection", None)
        if routing is None or not backend.computes_moba:
            continue
        assert_selection_matches(routing(q, k, cfg).cpu(), expected, backend.name)
        exercised += 1
    assert exercised >= 2  # ours and naive_torch


def _grads_oracle(q, k, v, g, cfg, sel, dtype, cu=None):
    qc, kc, vc, gc = (t.detach().cpu().to(dtype).requires_grad_(True) for t in (q, k, v, g))
    out = O.moba_attention(qc, kc, vc, oracle_cfg(cfg), selected=sel, query_chunk=256,
                           cu_seqlens=None if cu is None else cu.cpu())
    out.backward(gc.detach())
    return out.detach(), qc.grad, kc.grad, vc.grad


def _check_grads(got, truth, low):
    """The reference's policy (2x the bf16 oracle's own error), and the
    north star's bf16 bars; for dK / dV, which sum over every query of a
    kv head's group that selected the key, the bars scale with max|truth|."""
    for name, ours, tr, lo in zip(("out", "dq", "dk", "dv"), got, truth, low):
        assert_within_tolerance(ours, tr, max_abs_error(lo, tr), name)
        scale = max(1.0, tr.abs().max().item()) if name in ("dk", "dv") else 1.0
        assert max_abs_error(ours, tr) <= BF16_MAX_ABS * scale, name
        assert mean_abs_error(ours, tr) <= BF16_MEAN_ABS * scale, name


@pytest.mark.parametrize("shape,h_kv", [((1, 1024, 4, 64), 4), ((1, 1024, 8, 128), 2)])
def test_ours_forward_grad_matches_oracle_autograd(device, shape, h_kv):
    cfg = MoBAConfig(block_size=64, top_k=4, dtype=torch.bfloat16)
    q, k, v = make_qkv(shape, torch.bfloat16, seed=21, device=device)
    k, v = k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous()
    g = make_qkv(shape, torch.bfloat16, seed=22, device=device, n=1)[0]
    sel = oracle_selection(q, k, cfg)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = get_backend("ours").forward_grad(qq, kk, vv, cfg)
    out.backward(g)
    truth = _grads_oracle(q, k, v, g, cfg, sel, torch.float64)
    low = _grads_oracle(q, k, v, g, cfg, sel, torch.bfloat16)
    _check_grads((out, qq.grad, kk.grad, vv.grad), truth, low)


def _packed(device, lens, h, h_kv, d, seed):
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    t = int(cu[-1])
    q = make_qkv((1, t, h, d), torch.bfloat16, seed=seed, device=device, n=1)[0]
    k, v = make_qkv((1, t, h_kv, d), torch.bfloat16, seed=seed + 1, device=device, n=2)
    return q, k, v, cu.to(device)


def test_ours_forward_packed_matches_oracle(device):
    cfg = MoBAConfig(block_size=32, top_k=4, dtype=torch.bfloat16)
    q, k, v, cu = _packed(device, [300, 96, 513, 64], 4, 2, 64, seed=31)
    out = get_backend("ours").forward_packed(q, k, v, cfg, cu)
    sel = oracle_selection(q, k, cfg, cu_seqlens=cu)
    truth, ref_err = fp64_truth(q, k, v, cfg, sel, cu_seqlens=cu)
    assert_within_tolerance(out, truth, ref_err, "forward_packed")
    assert max_abs_error(out, truth) <= BF16_MAX_ABS


@pytest.mark.parametrize("h,h_kv,d", [(4, 4, 64), (8, 2, 128)])
def test_moba_attn_varlen_triton_forward_and_backward(device, h, h_kv, d):
    """The packed [T, H, D] signature: output and gradients against fp64
    autograd of the oracle, routing checked exactly."""
    lens = [640, 128, 1000, 256]
    q, k, v, cu = _packed(device, lens, h, h_kv, d, seed=41)
    g = make_qkv(q.shape, torch.bfloat16, seed=43, device=device, n=1)[0]
    cfg = MoBAConfig(block_size=64, top_k=4, dtype=torch.bfloat16)
    sel = oracle_selection(q, k, cfg, cu_seqlens=cu)
    qq, kk, vv = (t[0].clone().requires_grad_(True) for t in (q, k, v))
    out = moba_attn_varlen_triton(qq, kk, vv, cu, max(lens), 64, 4)
    assert out.shape == qq.shape and out.dtype is torch.bfloat16
    out.backward(g[0])
    truth = _grads_oracle(q, k, v, g, cfg, sel, torch.float64, cu=cu)
    low = _grads_oracle(q, k, v, g, cfg, sel, torch.bfloat16, cu=cu)
    got = (out.unsqueeze(0), qq.grad.unsqueeze(0), kk.grad.unsqueeze(0), vv.grad.unsqueeze(0))
    _check_grads(got, truth, low)


def test_moba_attn_varlen_triton_rejects_unpacked_input(device):
    q = torch.zeros(1, 128, 2, 64, dtype=torch.bfloat16, device=device)
    cu = torch.tensor([0, 128], dtype=torch.int32, device=device)
    with pytest.raises(ValueError, match="packed"):
        moba_attn_varlen_triton(q, q, q, cu, 128, 64, 4)
