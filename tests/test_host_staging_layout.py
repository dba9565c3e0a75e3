"""Layout of the pinned / device staging arenas for host-resident parameters
(gefen/host_staging.py), checked on the host: every piece 256-byte aligned,
the written pieces (parameter, then state) before the gradients so one copy
back covers exactly them, and chunks cut at the byte limit with an oversized
parameter alone in its chunk."""
import torch

from gefen import host_staging as hs


def _item(name, shape, dtype, factored, period):
    p = torch.zeros(shape, dtype=dtype)
    n = p.numel()
    state = {"m_codebook": torch.zeros(n // period, period, dtype=torch.uint8),
             "m_magnitude": torch.zeros(n // period, 1)}
    if factored:
        state["v_row"], state["v_col"] = torch.zeros(shape[0]), torch.zeros(shape[1])
    else:
        state["vmean"] = torch.zeros(n // period, 1)
    return hs.StagedItem(None, name, p, torch.zeros_like(p), factored, (state, 0.0, 1.0, 1.0, 1.0, 0.0))


def test_chunk_layout_written_region_first_and_aligned():
    items = [_item("a", (40, 64), torch.bfloat16, True, 64), _item("b", (300,), torch.float32, False, 100),
             _item("c", (24, 40), torch.float16, True, 8)]
    (chunk,) = hs.HostStager.chunks(items, 1 << 30)
    spans = []
    for it in items:
        keys = [k for k, _, _ in it.pieces]
        assert keys == ["p"] + list(it.state_keys())
        for _, t, off in it.pieces:
            assert off % 256 == 0
            spans.append((off, off + t.numel() * t.element_size()))
            assert off + t.numel() * t.element_size() <= chunk.written
        assert it.grad_offset % 256 == 0 and it.grad_offset >= chunk.written
        spans.append((it.grad_offset, it.grad_offset + it.grad.numel() * it.grad.element_size()))
    spans.sort()
    for (a0, a1), (b0, b1) in zip(spans, spans[1:]):
        assert a1 <= b0  # no overlap
    assert spans[-1][1] <= chunk.total
    assert sum(it.nbytes() for it in items) == chunk.total


def test_chunks_cut_at_the_limit():
    items = [_item("x%d" % i, (32, 32), torch.bfloat16, True, 32) for i in range(5)]
    per = items[0].nbytes()
    chunks = hs.HostStager.chunks(items, 2 * per)
    assert [len(c.items) for c in chunks] == [2, 2, 1]
    big = _item("big", (256, 256), torch.float32, True, 256)
    chunks = hs.HostStager.chunks([items[0], big, items[1]], 2 * per)
    assert [[it.name for it in c.items] for c in chunks] == [["x0"], ["big"], ["x1"]]


def test_pack_and_unpack_round_trip_through_a_host_arena():
    """The slices the packer and unpacker use address the same bytes."""
    it = _item("a", (8, 16), torch.bfloat16, True, 16)
    it.p.copy_(torch.arange(128, dtype=torch.float32).view(8, 16))
    (chunk,) = hs.HostStager.chunks([it], 1 << 20)
    arena = torch.zeros(chunk.total, dtype=torch.uint8)
    for _, t, off in it.pieces:
        hs._slice(arena, off, t).copy_(t)
    p_in_arena = hs._slice(arena, it.pieces[0][2], it.p)
    assert torch.equal(p_in_arena, it.p)
    p_in_arena.add_(1)
    it.p.zero_()
    hs.HostStager._unpack(chunk, arena, type("Done", (), {"synchronize": lambda self: None})())
    assert torch.equal(it.p.float(), torch.arange(128, dtype=torch.float32).view(8, 16) + 1)


def test_chunk_limit_from_the_environment(monkeypatch):
    monkeypatch.delenv("GEFENX_HOST_STAGING_BYTES", raising=False)
    assert hs.chunk_bytes_from_env() == hs.DEFAULT_CHUNK_BYTES
    monkeypatch.setenv("GEFENX_HOST_STAGING_BYTES", "4096")
    assert hs.chunk_bytes_from_env() == 4096
