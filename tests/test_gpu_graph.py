"""The whole fwd+bwd step captured in one HIP graph and replayed.

Every stage launches on the current stream, allocates through torch (a
graph-private pool during capture), clears memory with fill kernels rather
than hipMemsetAsync, and never synchronises the host on the padded path, so
`torch.cuda.graph` can capture `moba_attention` with its backward. Each
replay gets new inputs; eager runs of the same inputs go in between, and the
replay must reproduce them bit for bit (every stage is deterministic given
its inputs, the CSC column order included)."""

import pytest
import torch

from conftest import make_qkv
from moba.config import MoBAConfig
from moba.kernels.attention import moba_attention

pytestmark = pytest.mark.gpu


def step(q, k, v, g, cfg):
    out = moba_attention(q, k, v, cfg)
    dq, dk, dv = torch.autograd.grad(out, (q, k, v), g)
    return out, dq, dk, dv


@pytest.mark.parametrize("shape,h_kv,bs,tk", [((1, 4096, 4, 64), 4, 128, 8),
                                             ((2, 2048, 4, 64), 2, 64, 5)])
def test_fwd_bwd_replays_match_eager(device, shape, h_kv, bs, tk):
    cfg = MoBAConfig(block_size=bs, top_k=tk)

    def inputs(seed):
        q, k, v = make_qkv(shape, torch.bfloat16, seed=seed, device=device)
        g = make_qkv(shape, torch.bfloat16, seed=seed + 100, device=device, n=1)[0]
        return q, k[:, :, :h_kv].contiguous(), v[:, :, :h_kv].contiguous(), g

    q0, k0, v0, g0 = inputs(1)
    qs, ks, vs = (t.clone().requires_grad_(True) for t in (q0, k0, v0))
    gs = g0.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the capture stream
        for _ in range(2):
            step(qs, ks, vs, gs, cfg)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step(qs, ks, vs, gs, cfg)
    for seed in (11, 12, 13):
        q, k, v, g = inputs(seed)
        with torch.no_grad():
            qs.copy_(q)
            ks.copy_(k)
            vs.copy_(v)
            gs.copy_(g)
        graph.replay()
        torch.cuda.synchronize()
        eager = step(*(t.clone().requires_grad_(True) for t in (q, k, v)), g, cfg)
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "dq", "dk", "dv"), captured, eager):
            assert torch.equal(a, b), f"replay {seed}: {name} differs from eager"
