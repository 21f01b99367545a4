"""Host-side API behaviour that needs no GPU: config semantics, the backend
registry contract, validation errors, and the no-CPU-fallback rule."""

import pytest
import torch

import implementations
from implementations.base import Backend, get_backend, register
from moba.config import MoBAConfig
from moba.gqa import expand_kv, head_group_size
from moba.kernels.moba_fwd import _validate, moba_forward
from moba.varlen import validate_cu_seqlens


def test_config_defaults_and_budget():
    cfg = MoBAConfig(block_size=128, top_k=8)
    assert cfg.dtype is torch.bfloat16
    assert cfg.always_select_current and cfg.top_k_includes_current
    assert cfg.tie_break_low_index and not cfg.pool_masked_only
    assert cfg.past_blocks_selected(512) == 7
    assert cfg.past_blocks_selected(3) == 3
    assert cfg.num_blocks(1000) == 8
    assert cfg.slots() == 8
    assert MoBAConfig(32, 3, top_k_includes_current=False).slots() == 4
    assert MoBAConfig(32, 3, always_select_current=False).slots() == 3
    with pytest.raises(ValueError):
        MoBAConfig(block_size=0, top_k=1)
    with pytest.raises(ValueError):
        MoBAConfig(block_size=16, top_k=0)
    with pytest.raises(Exception):
        cfg.top_k = 3  # frozen


def test_head_group_and_expand():
    assert head_group_size(32, 8) == 4
    with pytest.raises(ValueError):
        head_group_size(6, 4)
    t = torch.arange(2 * 3).view(1, 1, 2, 3)
    e = expand_kv(t, 4)
    assert torch.equal(e[0, 0, :, 0], torch.tensor([0, 0, 3, 3]))


def test_registry_contract():
    names = [b.name for b in implementations.all_backends()]
    assert {"ours", "naive_torch", "sdpa_dense"} <= set(names)
    # The vendored third-party name is not claimed by this build's kernels.
    assert "triton_moba" not in names
    assert get_backend("ours").computes_moba and not get_backend("sdpa_dense").computes_moba
    cfg = MoBAConfig(block_size=128, top_k=8)
    for b in implementations.all_backends():
        assert isinstance(b, Backend)
        ok, reason = b.is_available(cfg)  # never raises
        assert isinstance(ok, bool) and isinstance(reason, str)
        if not torch.cuda.is_available() and b.name != "naive_torch":
            assert not ok and reason
    with pytest.raises(ValueError):
        register(get_backend("ours"))
    with pytest.raises(KeyError, match="ours"):
        get_backend("nope")


def test_validation_errors():
    cfg = MoBAConfig(block_size=128, top_k=8)
    q = torch.zeros(1, 256, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="key/value"):
        _validate(q, q, q[:, :, :2], cfg)
    with pytest.raises(ValueError, match="divisible"):
        _validate(q, q[:, :, :3], q[:, :, :3], cfg)
    with pytest.raises(ValueError, match="power of two"):
        z = torch.zeros(1, 256, 4, 96, dtype=torch.bfloat16)
        _validate(z, z, z, cfg)
    with pytest.raises(ValueError, match="cache line"):
        z = torch.zeros(1, 256, 4, 32, dtype=torch.bfloat16)
        _validate(z, z, z, cfg)
    with pytest.raises(ValueError, match="block_size"):
        _validate(q, q, q, MoBAConfig(block_size=8, top_k=2))
    with pytest.raises(ValueError, match="max_seqlen"):
        _validate(q, q, q, cfg, cu_seqlens=torch.tensor([0, 256], dtype=torch.int32))


def test_cu_seqlens_validation():
    good = torch.tensor([0, 80, 128, 212], dtype=torch.int32)
    assert validate_cu_seqlens(good, 212, 84) == 3
    with pytest.raises(ValueError, match="int32"):
        validate_cu_seqlens(good.long(), 212, 84)
    with pytest.raises(ValueError, match="start at 0"):
        validate_cu_seqlens(torch.tensor([1, 212], dtype=torch.int32), 212, 300)
    with pytest.raises(ValueError, match="increasing"):
        validate_cu_seqlens(torch.tensor([0, 80, 80, 212], dtype=torch.int32), 212, 200)
    with pytest.raises(ValueError, match="ends at"):
        validate_cu_seqlens(good, 300, 84)
    with pytest.raises(ValueError, match="below the longest"):
        validate_cu_seqlens(good, 212, 50)


def test_no_cpu_fallback():
    """The product path never computes on the CPU: CPU tensors are refused."""
    cfg = MoBAConfig(block_size=128, top_k=8)
    q = torch.zeros(1, 256, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        moba_forward(q, q, q, cfg)


def test_index_stride_layouts():
    """The index arrays reach the library as (base pointer, element stride):
    3 for the (row, head, slot) records the CSC build makes, 1 for three
    separate arrays; anything else is refused before a launch."""
    from moba.kernels.routing import CSCIndex, index_stride

    def make(rows, heads, slots):
        z = torch.zeros(1, 2, 8, dtype=torch.int32)
        return CSCIndex(col_nnz=z, col_offsets=z, row_indices=rows, head_indices=heads,
                        slot_of_pair=slots, order=z, num_blocks=8, max_slots=2,
                        num_query_heads=2)

    rec = torch.zeros(1, 2, 16, 3, dtype=torch.int32)
    r, h, s = rec.unbind(-1)
    assert index_stride(make(r, h, s)) == 3
    assert h.data_ptr() - r.data_ptr() == 4 and s.data_ptr() - r.data_ptr() == 8
    sep = [torch.zeros(1, 2, 16, dtype=torch.int32) for _ in range(3)]
    assert index_stride(make(*sep)) == 1
    with pytest.raises(ValueError):
        index_stride(make(r, sep[1], sep[2]))           # mixed strides
    with pytest.raises(ValueError):
        index_stride(make(*(t.long() for t in sep)))   # wrong dtype
    wide = [torch.zeros(1, 2, 20, dtype=torch.int32)[:, :, :16] for _ in range(3)]
    with pytest.raises(ValueError):
        index_stride(make(*wide))                      # padding between kv heads
    even = [t[:, :, ::2] for t in sep]                 # uniform stride 2 is fine
    assert index_stride(make(*even)) == 2


@pytest.mark.parametrize("batch,h_kv,group,budget", [(1, 4, 1, 100), (2, 4, 1, 8), (3, 4, 1, 4),
                                                    (2, 4, 1, 3), (2, 8, 1, 1), (1, 1, 1, 0),
                                                    (2, 2, 4, 0.5), (1, 3, 8, 0.25), (1, 2, 8, 0.3),
                                                    (2, 2, 4, 0)])
def test_partials_chunk_plan(batch, h_kv, group, budget):
    """Every (batch row, query head) lands in exactly one chunk, chunks stay
    within the budget unless one query head of one row alone exceeds it, a
    chunk splits a kv head's group only when it holds that kv head alone,
    and a budget that holds everything gives a single chunk."""
    from moba.chunking import plan_chunks, query_heads

    unit = 1000 * group  # bytes of one (row, kv head) unit: `group` query heads
    chunks = plan_chunks(batch, h_kv, unit, int(budget * unit), group=group)
    seen = [(b, h) for c in chunks for b in range(c[0], c[1])
            for h in range(*query_heads(c, group))]
    assert sorted(seen) == [(b, h) for b in range(batch) for h in range(h_kv * group)]
    for b0, b1, h0, h1, j0, j1 in chunks:
        heads = (h1 - h0) * group if (j0, j1) == (0, group) else j1 - j0
        assert (b1 - b0) * heads * (unit // group) <= max(unit // group, budget * unit)
        assert b1 - b0 == 1 or (h0, h1) == (0, h_kv)   # rectangles: whole rows or one row
        assert (j0, j1) == (0, group) or h1 - h0 == 1  # a split group: one kv head
    if budget >= batch * h_kv:
        assert chunks == [(0, batch, 0, h_kv, 0, group)]


def test_chunk_plan_sizes_packed_units_by_total_tokens():
    """Packed input keeps [1, Hq, T, slots, D] partials: a unit is all T
    tokens of the one row, not max_seqlen of them."""
    from moba.chunking import plan_call, unit_bytes
    t, max_seqlen, h, d, slots = 524288, 32768, 4, 64, 8
    unit = unit_bytes(t, 1, d, slots, 2)
    assert unit == t * slots * (d * 2 + 8)
    # Budget fits one kv head's T-token unit but not two: one chunk per head.
    chunks = plan_call((1, t, h, d), h, slots, 2, budget=unit + unit // 2)
    assert chunks == [(0, 1, hk, hk + 1, 0, 1) for hk in range(h)]
    # Sized by max_seqlen (16x too small) it would have taken one chunk.
    assert 4 * unit_bytes(max_seqlen, 1, d, slots, 2) <= unit + unit // 2
    # float32 part_acc doubles the value rows.
    assert plan_call((1, t, h, d), h, slots, 4, budget=unit + unit // 2) == \
        [(0, 1, hk, hk + 1, 0, 1) for hk in range(h)]
    assert len(plan_call((1, t, h, d), h, slots, 4, budget=2 * unit)) == 4


def test_hierarchical_gate_config_fields():
    cfg = MoBAConfig(block_size=128, top_k=8)
    assert cfg.gate_group == 0 and cfg.gate_open == 0  # exact gate by default
    MoBAConfig(block_size=128, top_k=8, gate_group=16, gate_open=8)
    with pytest.raises(ValueError, match="gate_open"):
        MoBAConfig(block_size=128, top_k=8, gate_group=16)
    with pytest.raises(ValueError, match="non-negative"):
        MoBAConfig(block_size=128, top_k=8, gate_group=-1, gate_open=2)


def test_validation_head_dim_range():
    cfg = MoBAConfig(block_size=128, top_k=8)
    for d in (256, 512, 1024):  # the FMA kernels, keys staged in tiles past 256
        z = torch.zeros(1, 256, 2, d, dtype=torch.bfloat16)
        _validate(z, z, z, cfg)
    with pytest.raises(ValueError, match="above 1024"):
        z = torch.zeros(1, 256, 2, 2048, dtype=torch.bfloat16)
        _validate(z, z, z, cfg)


@pytest.mark.parametrize("dtype,d,bs,ok", [
    (torch.float32, 256, 128, True),    # 256 KiB of keys and values: tiles of keys
    (torch.bfloat16, 256, 256, True),
    (torch.float32, 1024, 512, True),
    (torch.float32, 1024, 2048, False),  # 16 score rows of 2048 alone exceed LDS
    (torch.bfloat16, 128, 128, True),   # MFMA kernel
])
def test_validation_rejects_blocks_beyond_lds(dtype, d, bs, ok):
    """The FMA attend kernel stages a block's keys and values in tiles when
    they do not fit in LDS whole, but a group's 16 query rows and score rows
    must fit: a shape beyond that is a ValueError before any launch, not a
    failure inside the library call."""
    cfg = MoBAConfig(block_size=bs, top_k=2, dtype=dtype)
    z = torch.zeros(1, 4 * bs, 2, d, dtype=dtype)
    if ok:
        _validate(z, z, z, cfg)
    else:
        with pytest.raises(ValueError, match="LDS"):
            _validate(z, z, z, cfg)
