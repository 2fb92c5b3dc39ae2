"""Host-side logic of the product path that runs without a GPU, checked against the oracle."""
from __future__ import annotations

import pytest
import torch

import oracle.reference_cpu as ref
from semblo_amd.token_outer_prefill import reserved_layout


def _layout_or_none(fn, *args):
    try:
        return fn(*args)
    except RuntimeError:
        return None


@pytest.mark.parametrize("align", [1, 16, 64])
def test_reserved_layout_matches_the_oracle_bit_for_bit(align):
    """The host computes every KV head's layout in whole-array arithmetic; the runs
    must come out exactly as the oracle's per-head restatement lays them out
    (token_outer_prefill.py:39-63), and refuse the same stores."""
    g = torch.Generator().manual_seed(align)
    refused = 0
    for t in range(300):
        hkv = int(torch.randint(1, 9, (1,), generator=g))
        c = int(torch.randint(3, 600, (1,), generator=g))
        if t % 3 == 0:
            sizes = torch.randint(0, 3000, (hkv, c), generator=g)
        elif t % 3 == 1:                         # a few large clusters, many tiny ones
            sizes = (torch.rand(hkv, c, generator=g) ** 8 * 5000).long()
        else:                                    # nearly every cluster empty
            sizes = torch.zeros(hkv, c, dtype=torch.long)
            sizes[:, :3] = torch.randint(0, 99999, (hkv, 3), generator=g)
        n = int(sizes.sum(1).max()) + int(torch.randint(0, 50, (1,), generator=g))
        total = n * int(torch.randint(1, 8, (1,), generator=g)) + int(torch.randint(0, 1000, (1,), generator=g))
        width = total + c * align + int(torch.randint(-3000, 5000, (1,), generator=g))
        want = _layout_or_none(ref.reserved_layout, sizes, n, total, width, align)
        got = _layout_or_none(reserved_layout, sizes, n, total, width, align)
        refused += want is None
        assert (want is None) == (got is None), (t, hkv, c, width)
        if want is not None:
            assert got.dtype == torch.int64 and torch.equal(got, want), (t, hkv, c, width)
    assert 0 < refused < 300          # both outcomes were exercised


def test_streamed_queries_refuse_a_slice_past_the_prompt():
    """StreamedPrefillSession.queries refuses positions outside [0, tokens) before it
    touches a device (model.py:1509-1524 takes slices inside the prompt only)."""
    import types
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.streamed_prefill import StreamedPrefillSession
    cfg = SembloRuntimeConfig(num_q_heads=4, num_kv_heads=1, head_dim=64)
    layer = types.SimpleNamespace(runtime_config=cfg, num_heads=4, num_kv_heads=1, head_dim=64,
                                  target_tokens=0, index=None, arena=None)
    session = StreamedPrefillSession(layer, 100)
    session.index = object()                 # past ingest
    q = torch.zeros(8, 4, 64, dtype=torch.bfloat16)
    for start in (95, -1, 100):
        with pytest.raises(ValueError, match="outside the prompt"):
            session.attend(q, q, start)


def test_sessions_driven_by_hidden_states_need_projections_and_a_prompt_from_zero():
    """A session driven by hidden states runs the model's projections, which the
    model attaches to the layer: without them it refuses.  Positions given to
    begin_* must run 0 .. T-1, as a [T] row or an M-RoPE grid [3, T]."""
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.model import SembloAttention
    cfg = SembloRuntimeConfig(num_q_heads=4, num_kv_heads=1, head_dim=64)
    layer = SembloAttention(cfg, layer_name="host.hidden")
    session = layer.begin_streamed_prefill(torch.arange(256))
    assert session.tokens == 256
    with pytest.raises(RuntimeError, match="no projections"):
        session.keys(torch.arange(0, 64), torch.zeros(64, 32), 0, 64)
    grid = torch.arange(300).expand(3, 300)
    assert layer.begin_streamed_prefill(grid).tokens == 300
    token = layer.begin_token_outer_prefill(grid, 64)
    assert token.tokens == 300 and token.rope_positions.shape == (3, 300)
    with pytest.raises(RuntimeError, match="no projections"):
        token.slice(torch.zeros(64, 32), 0, 64)
    with pytest.raises(ValueError, match="0 .. T-1"):
        layer.begin_streamed_prefill(torch.arange(5, 261))
    rope, flat = layer._positions_for_runtime(grid)
    assert rope is grid and torch.equal(flat, torch.arange(300))
    assert torch.equal(layer._slice_positions(grid, 10, 20), grid[:, 10:20])
    calls = []
    layer.attach_projections(lambda p, h: calls.append(("qkv", p)) or (None,) * 6, lambda a, g: a)
    with pytest.raises(RuntimeError, match="its own K/V"):
        session.keys(torch.arange(0, 64), torch.zeros(64, 32), 0, 64)
    assert calls and calls[0][0] == "qkv"


def test_capacity_arena_adopts_in_place_with_empty_tail_clusters():
    """DecodeArena.with_capacity / adopt on CPU tensors (arena.py:66-253 of the
    reference): before any request a one-token index with the prompt length at the
    capacity; an adopted index fills the first clusters, the rest are empty runs with
    zero descriptors, the suffix table maps the blocks from the prompt's end, and no
    buffer moves.  An index larger than the arena is refused."""
    import types
    from semblo_amd.arena import DecodeArena
    hkv, d, cap, ncl = 2, 8, 1000, 16
    arena = DecodeArena.with_capacity(capacity=cap, num_kv_heads=hkv, head_dim=d, num_clusters=ncl,
                                      reserve=300, suffix_block=64, dtype=torch.float32, device="cpu")
    assert arena.reads_prompt_length_on_device and int(arena.prompt_length_t) == cap
    assert arena.sizes[:, 0].tolist() == [1, 1] and int(arena.sizes[:, 1:].sum()) == 0
    assert arena.indptr[:, 1:].eq(1).all()
    ptrs = [t.data_ptr() for t in (arena.codebooks, arena.sizes, arena.indptr, arena.packed_kv,
                                   arena.suffix_kv, arena.suffix_table, arena.prompt_length_t)]
    c, length = 5, 700
    sizes = torch.tensor([[100, 0, 300, 250, 50], [140, 140, 140, 140, 140]], dtype=torch.int32)
    padded = (sizes + 15) // 16 * 16
    indptr = torch.zeros(hkv, c + 1, dtype=torch.int32)
    indptr[:, 1:] = padded.cumsum(1)
    rows = int(indptr[:, -1].max()) + 40
    index = types.SimpleNamespace(
        bucket_sizes=sizes, bucket_indptr=indptr, prompt_length=length,
        codebooks=torch.randn(hkv, 2, c, d // 2), packed_kv=torch.randn(2, rows, hkv, d),
        posting_positions=torch.randint(0, length, (hkv, rows), dtype=torch.int32))
    arena.adopt(index)
    assert [t.data_ptr() for t in (arena.codebooks, arena.sizes, arena.indptr, arena.packed_kv,
                                   arena.suffix_kv, arena.suffix_table, arena.prompt_length_t)] == ptrs
    assert torch.equal(arena.sizes[:, :c], sizes) and int(arena.sizes[:, c:].abs().sum()) == 0
    assert torch.equal(arena.indptr[:, :c + 1], indptr)
    assert torch.equal(arena.indptr[:, c + 1:], indptr[:, c:c + 1].expand(hkv, ncl - c))
    assert torch.equal(arena.codebooks[:, :, :c], index.codebooks)
    assert int(arena.codebooks[:, :, c:].abs().sum()) == 0
    assert torch.equal(arena.packed_kv[:, :rows], index.packed_kv)
    assert int(arena.prompt_length_t) == length and arena.prompt_length == length
    # positions 700 .. 999 (the reserve) land in distinct physical blocks from block 10 on
    blocks = torch.arange(length, length + 300) // 64
    phys = arena.suffix_table[blocks]
    assert phys[0] == 0 and len(set(phys.tolist())) == int(blocks[-1] - blocks[0]) + 1
    assert int(phys.max()) < arena.suffix_kv.shape[1]
    assert int(arena.suffix_table[:length // 64].abs().sum()) == 0
    big = types.SimpleNamespace(**{**vars(index), "prompt_length": cap + 1})
    with pytest.raises(ValueError, match="arena holds 1000"):
        arena.adopt(big)
    many = types.SimpleNamespace(**{**vars(index), "bucket_sizes": torch.ones(hkv, ncl + 1, dtype=torch.int32)})
    with pytest.raises(ValueError, match="clusters"):
        arena.adopt(many)


def test_decode_budget_is_chosen_per_step(monkeypatch):
    """Decode selects on its own budget when SEMBLO_DECODE_TARGET_TOKENS sets one
    (tests/test_decode_only_budget.py of the reference), else on the last prefill's,
    else with a capacity arena on the budget at the capacity; a prefill's budget is
    left as it was (model.py:847-854)."""
    from semblo_amd.config import SembloRuntimeConfig
    from semblo_amd.model import SembloAttention
    monkeypatch.delenv("SEMBLO_DECODE_TARGET_TOKENS", raising=False)
    cfg = SembloRuntimeConfig(num_q_heads=4, num_kv_heads=1, head_dim=64)
    assert cfg.decode_target_tokens == 0
    layer = SembloAttention(cfg, layer_name="host.budget.a")
    layer.target_tokens = cfg.budget(65536)            # what a prefill of 65536 sets
    assert layer.decode_budget() == 4096
    monkeypatch.setenv("SEMBLO_DECODE_TARGET_TOKENS", "524288")
    cfg = SembloRuntimeConfig(num_q_heads=4, num_kv_heads=1, head_dim=64)
    layer = SembloAttention(cfg, layer_name="host.budget.b")
    layer.target_tokens = cfg.budget(65536)
    assert layer.decode_budget() == 524288
    assert layer.target_tokens == 4096, "the prefill keeps its budget"
    monkeypatch.delenv("SEMBLO_DECODE_TARGET_TOKENS")
    cfg = SembloRuntimeConfig(num_q_heads=4, num_kv_heads=1, head_dim=64, decode_capacity=131072)
    layer = SembloAttention(cfg, layer_name="host.budget.c")
    layer.target_tokens = cfg.budget(2048)
    assert layer.decode_budget() == 8192


def test_flush_range_keeps_the_newest_and_moves_the_rest():
    """suffix_flush.flush_range (suffix_flush.py:140-152 of the reference), the cases of
    its own test: once the exact suffix holds keep + every tokens, everything but the
    newest ``keep`` moves, from the current prompt length on; an empty range moves
    nothing."""
    from semblo_amd.suffix_flush import flush_layer, flush_range
    length, keep, every = 1000, 100, 50
    plen, moved = length, []
    for written in range(400):
        assert length + written - plen < keep + every + 1
        r = flush_range(length, written, plen, keep, every)
        if r is not None:
            frm, to = r
            assert frm == plen and to == length + written - keep and to - frm >= every
            moved.append(r)
            plen = to
    assert moved and moved[0] == (length, length + 50)
    assert all(b - a == every for a, b in moved)
    assert flush_range(length, 10 ** 6, length, keep, 0) is None          # flush off
    assert flush_layer(object(), 1200, 1200) == 0                         # nothing to move
