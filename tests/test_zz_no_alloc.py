"""moba_gate_noalloc (static device scratch, no workspace argument) against
moba_gate (caller workspace), called through the C ABI: ids bit-exact, on
consecutive calls whose second input is smaller, so the second call runs on
scratch the first one left behind."""

import pytest
import torch

from conftest import make_qkv
from moba import _lib
from moba.config import MoBAConfig
from moba.kernels.pooling import pool_blocks

pytestmark = pytest.mark.gpu


def _gate_args(q, kbar, cfg, out):
    b, s, h, d = q.shape
    take = cfg.past_blocks_selected(kbar.shape[2])
    return [_lib.ptr(q), _lib.ptr(kbar), _lib.ptr(out), None, b, s, s, h, kbar.shape[1], d,
            kbar.shape[2], cfg.block_size, cfg.slots(), take,
            int(bool(cfg.always_select_current)), _lib.DTYPE_CODE[q.dtype]]


def _both(q, k, cfg):
    dev = q.device
    kbar = pool_blocks(k, cfg)
    b, s, h, _ = q.shape
    ref = torch.full((b, h, s, cfg.slots()), -7, device=dev, dtype=torch.int32)
    got = torch.full_like(ref, -9)
    lib = _lib.load()
    ws = torch.empty(int(lib.moba_gate_workspace_size(b, s, h)), device=dev, dtype=torch.uint8)
    stream = _lib.stream_handle(dev)
    _lib.call("moba_gate", *_gate_args(q, kbar, cfg, ref), _lib.ptr(ws), ws.numel(), stream)
    _lib.call("moba_gate_noalloc", *_gate_args(q, kbar, cfg, got), stream)
    torch.cuda.synchronize()
    return ref.cpu(), got.cpu()


def _check(q, k, cfg, label):
    print(f"[no_alloc] {label} shape={tuple(q.shape)} dtype={q.dtype} "
          f"bs={cfg.block_size} k={cfg.top_k}", flush=True)
    ref, got = _both(q, k, cfg)
    bad = (ref != got).any(-1)
    assert not bool(bad.any()), (
        f"{label}: {int(bad.sum())} queries differ; first {torch.nonzero(bad)[0].tolist()}")
    assert int((ref == -7).sum()) == 0, f"{label}: moba_gate left slots unwritten"


def test_noalloc_matches_workspace_gate_twice(device):
    # First call: integer-valued inputs make exact ties, so undecidable
    # queries go through the queue held in the static scratch.
    cfg = MoBAConfig(block_size=128, top_k=8, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(3)
    shape = (1, 16384, 4, 64)
    q = torch.randint(-2, 3, shape, generator=g).to(torch.bfloat16).to(device)
    k = torch.randint(-2, 3, shape, generator=g).to(torch.bfloat16).to(device)
    _check(q, k, cfg, "call 1 (ties)")
    # Second call, smaller: the scratch still holds call 1's counter, norms
    # and queue; the call must clear what it relies on.
    cfg2 = MoBAConfig(block_size=64, top_k=4, dtype=torch.bfloat16)
    q2, k2, _ = make_qkv((1, 4096, 2, 64), torch.bfloat16, seed=5, device=device)
    _check(q2, k2, cfg2, "call 2 (smaller)")


def test_noalloc_gqa_fp16_then_headline_shape(device):
    cfg = MoBAConfig(block_size=128, top_k=8, dtype=torch.float16)
    q, _, _ = make_qkv((1, 8192, 8, 128), torch.float16, seed=1, device=device)
    _, k, _ = make_qkv((1, 8192, 2, 128), torch.float16, seed=2, device=device)
    _check(q, k, cfg, "gqa fp16")
    # The largest shape the scratch admits: [1, 512K, 4, 64] is 2^21 query rows.
    cfg = MoBAConfig(block_size=128, top_k=8, dtype=torch.bfloat16)
    q, k, _ = make_qkv((1, 524288, 4, 64), torch.bfloat16, seed=0, device=device)
    _check(q, k, cfg, "headline")
    # A smaller call after the largest one.
    q, k, _ = make_qkv((1, 2048, 1, 64), torch.bfloat16, seed=4, device=device)
    _check(q, k, MoBAConfig(block_size=32, top_k=8, dtype=torch.bfloat16), "small after large")


def test_noalloc_rejects_oversized(device):
    lib = _lib.load()
    # 2^21 + 1024 query rows: one block past the limit, rejected on the host.
    rc = lib.moba_gate_noalloc(None, None, None, None, 1, 524288 + 256, 524288 + 256, 4, 4,
                               64, 4099, 128, 8, 7, 1, 0, None)
    assert rc == _lib.MOBA_ERR_WORKSPACE
    assert b"static scratch limit" in lib.moba_last_error()


def test_noalloc_replays_in_a_graph_match_the_oracle(device):
    """The callers this entry point is for capture it: one eager call first
    (it takes the scratch address on the device), then a capture of
    moba_gate_noalloc alone, replayed on new q / kbar copied into the
    captured buffers, with eager work in between; every replay's ids equal
    the C oracle's."""
    from oracle import c_oracle
    from conftest import oracle_cfg

    cfg = MoBAConfig(block_size=64, top_k=8, dtype=torch.bfloat16)
    shape = (1, 4096, 2, 64)
    q0, k0, _ = make_qkv(shape, torch.bfloat16, seed=40, device=device)
    qs, kbs = q0.clone(), pool_blocks(k0, cfg)
    out = torch.full((1, 2, shape[1], cfg.slots()), -9, device=device, dtype=torch.int32)
    args = _gate_args(qs, kbs, cfg, out)
    _lib.call("moba_gate_noalloc", *args, _lib.stream_handle(device))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.call("moba_gate_noalloc", *args, _lib.stream_handle(device))
    for seed in (41, 42, 43):
        q, k, _ = make_qkv(shape, torch.bfloat16, seed=seed, device=device)
        kb = pool_blocks(k, cfg)
        qs.copy_(q)
        kbs.copy_(kb)
        out.fill_(-9)
        graph.replay()
        torch.cuda.synchronize()
        want = c_oracle.gate_select(q.cpu(), kb.cpu(), oracle_cfg(cfg))
        bad = (out.cpu() != want).any(-1)
        assert not bool(bad.any()), f"replay {seed}: {int(bad.sum())} queries differ"
