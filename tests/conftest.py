"""Shared fixtures, markers and shape sweeps.

Inputs follow the reference's scheme (`tests/conftest.py:83-98`): one seeded
`torch.Generator`, q, k, v drawn in that order. They are drawn on the CPU and
moved, so the GPU tests and the CPU oracle see identical values.
"""

import math
import os
import sys
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "moba-triton_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

# (batch, seq_len, heads, head_dim) -- reference SHAPE_SWEEP (conftest.py:40-45)
SHAPE_SWEEP = [
    (1, 1024, 4, 128),
    (2, 1024, 4, 128),
    (1, 2048, 4, 128),
    (1, 2048, 4, 64),
]
LONG_SHAPE_SWEEP = [
    (1, 4096, 4, 128),
    (1, 4096, 4, 64),
    (1, 8192, 2, 128),
]
# (block_size, top_k) -- reference GATE_SWEEP (conftest.py:73-80)
GATE_SWEEP = [(32, 4), (32, 8), (64, 4), (64, 8), (128, 8), (128, 12)]
MIN_BLOCKS_PER_SELECTION = 4


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")
    config.addinivalue_line("markers", "slow: long-context shapes")


def make_qkv(shape, dtype=torch.float64, seed=0, device="cpu", n=3):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(shape, generator=g, dtype=torch.float32).to(dtype).to(device)
                 for _ in range(n))


def gate_is_sparse(shape, gate):
    return math.ceil(shape[1] / gate[0]) >= MIN_BLOCKS_PER_SELECTION * gate[1]


def sweep_cases(include_long=True):
    cases = []
    for shape in SHAPE_SWEEP:
        for gate in GATE_SWEEP:
            if gate_is_sparse(shape, gate):
                cases.append(pytest.param(shape, gate, id=case_id(shape, gate)))
    if include_long:
        for shape in LONG_SHAPE_SWEEP:
            for gate in GATE_SWEEP:
                if gate_is_sparse(shape, gate):
                    cases.append(pytest.param(shape, gate, id=case_id(shape, gate),
                                              marks=pytest.mark.slow))
    return cases


def case_id(shape, gate):
    b, s, h, d = shape
    return f"b{b}s{s}h{h}d{d}-blk{gate[0]}-top{gate[1]}"


def oracle_cfg(cfg):
    """The oracle's duck-typed view of a MoBAConfig."""
    return SimpleNamespace(block_size=cfg.block_size, top_k=cfg.top_k,
                           always_select_current=cfg.always_select_current,
                           top_k_includes_current=cfg.top_k_includes_current,
                           tie_break_low_index=cfg.tie_break_low_index)


@pytest.fixture(scope="session")
def device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU device")
    return "cuda"


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the case before any GPU work, flushed, so a fault still says where.
    if request.node.get_closest_marker("gpu"):
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
