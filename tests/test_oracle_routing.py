"""Pins the routing oracle: slot-major metadata, per-row depth tables and packed
address expansion give the same addresses by three routes; segment moves equal
slicing; gathers and scatters round-trip."""

import torch

from oracle import routing as orr


def _world(seed=0, slots=6, planes=4, width=9, page=16, nblocks=400):
    g = torch.Generator().manual_seed(seed)
    tables = torch.randperm(nblocks, generator=g)[: slots * planes * width]
    tables = tables.view(slots, planes, width).int()
    n = 12
    slot = torch.randint(0, slots, (n,), generator=g)
    depth = torch.randint(0, planes, (n,), generator=g)
    pos = torch.randint(0, width * page, (n,), generator=g)
    return g, tables, slot, depth, pos, page


def test_metadata_matches_per_row_depth_tables():
    _, tables, slot, depth, pos, page = _world()
    slots_, planes, width = tables.shape
    desc = torch.stack([slot, depth, pos], 1)
    m = orr.metadata(desc, tables.view(-1, width), 12, 16, width, page, planes, width)
    t, b, o, ln = orr.depth_tables(tables[slot], depth, pos, page)
    assert torch.equal(m["tables"][:12], t) and torch.equal(m["blocks"], b)
    assert torch.equal(m["offsets"], o) and torch.equal(m["lengths"][:12], ln)
    assert torch.equal(m["slots"][:12], slot) and torch.equal(m["positions"][:12], pos)
    # rows past count are zero (padding of a bucketed graph batch)
    assert not m["tables"][12:].any() and not m["lengths"][12:].any()


def test_metadata_single_plane_ignores_depth():
    _, tables, slot, depth, pos, page = _world(1, planes=1)
    width = tables.shape[2]
    desc = torch.stack([slot, depth + 3, pos], 1)
    m = orr.metadata(desc, tables.view(-1, width), 12, 12, width, page, 1, width)
    t, b, _, _ = orr.depth_tables(tables[slot], torch.zeros_like(depth), pos, page)
    assert torch.equal(m["tables"], t) and torch.equal(m["blocks"], b)


def test_expand_kv_addresses_matches_depth_tables():
    _, tables, slot, depth, pos, page = _world(2)
    t, b, o, _ = orr.depth_tables(tables[slot], depth, pos, page)
    seq = torch.arange(12, dtype=torch.int32)
    eb, eo = orr.expand_kv_addresses(pos, seq, t.contiguous(), 12, t.shape[1], page)
    assert torch.equal(eb, b) and torch.equal(eo, o)


def test_depth_tables_inactive_rows_have_zero_length():
    _, tables, slot, depth, pos, page = _world(3)
    active = torch.arange(12) % 3 != 0
    _, _, _, ln = orr.depth_tables(tables[slot], depth, pos, page, active)
    assert torch.equal(ln, torch.where(active, pos + 1, 0).int())


def test_segments_equal_slicing_and_round_trip():
    g = torch.Generator().manual_seed(4)
    states = torch.randn(5, 10, 7, generator=g)
    segs = torch.tensor([[0, 2, 3, 0, 1], [3, 0, 4, 3, 0], [4, 7, 3, 7, 1]])
    out = torch.zeros(10, 7)
    orr.gather_segments(states, segs, out, 4)
    want = torch.cat([states[0, 2:5], states[3, 0:4], states[4, 7:10]])
    assert torch.equal(out, want)
    back = torch.zeros_like(states)
    orr.scatter_segments(out, segs, back, 4)
    assert torch.equal(back[0, 2:5], states[0, 2:5]) and torch.equal(back[4, 7:10], states[4, 7:10])
    assert not back[3].any()  # keep = 0
    # max_rows truncates
    out2 = torch.zeros(10, 7)
    orr.gather_segments(states, segs, out2, 2)
    assert torch.equal(out2[0:2], states[0, 2:4]) and not out2[2].any()


def test_gather_scatter_rows_round_trip():
    g = torch.Generator().manual_seed(5)
    pool = torch.randn(20, 33, generator=g)
    ids = torch.randperm(20, generator=g)[:8]
    got = orr.gather_rows(pool, ids, 6, 8)
    assert torch.equal(got[:6], pool[ids[:6]]) and not got[6:].any()
    fresh = torch.zeros_like(pool)
    orr.scatter_rows(got, ids, fresh, 6)
    assert torch.equal(fresh[ids[:6]], pool[ids[:6]])
    assert int((fresh != 0).any(1).sum()) == 6
