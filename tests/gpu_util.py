"""Helpers shared by the GPU parity tests."""

import torch

from conftest import oracle_cfg
from oracle import naive as O


def to_cpu(*ts):
    return tuple(t.detach().cpu() for t in ts)


def oracle_selection(q, k, cfg, cu_seqlens=None):
    """Selection mask from the torch oracle on CPU copies of the inputs."""
    qc, kc = to_cpu(q, k)
    cu = None if cu_seqlens is None else cu_seqlens.cpu()
    return O.moba_selection(qc, kc, oracle_cfg(cfg), cu_seqlens=cu)


def fp64_truth(q, k, v, cfg, sel, cu_seqlens=None, query_chunk=256):
    """(truth, ref_error): fp64 oracle and the same oracle in cfg's dtype,
    selection held fixed (reference tests/tolerance.py:64-107)."""
    qc, kc, vc = to_cpu(q, k, v)
    cu = None if cu_seqlens is None else cu_seqlens.cpu()
    oc = oracle_cfg(cfg)
    truth = O.moba_attention(qc.double(), kc.double(), vc.double(), oc, selected=sel,
                             query_chunk=query_chunk, cu_seqlens=cu)
    low = O.moba_attention(qc, kc, vc, oc, selected=sel, query_chunk=query_chunk,
                           cu_seqlens=cu)
    return truth, (low.double() - truth).abs().max().item()
