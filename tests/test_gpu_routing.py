"""GPU parity of the device routing / metadata kernels against the oracle (bit for
bit: all integer or byte moves), including replay of captured HIP graphs with new
descriptor contents and descriptors in pinned host memory."""

import ctypes

import pytest
import torch

from oracle import routing as orr

pytestmark = pytest.mark.gpu


def _descriptors(g, count, slots, planes, width, page, bad=True):
    slot = torch.randint(0, slots, (count,), generator=g)
    depth = torch.randint(0, planes, (count,), generator=g)
    pos = torch.randint(0, width * page, (count,), generator=g)
    d = torch.stack([slot, depth, pos], 1)
    if bad and count >= 4:
        d[1, 0] = slots + 5          # slot outside the tables
        d[2, 2] = width * page + 40  # position beyond the table
        d[3, 1] = planes + 2         # depth beyond the planes (ignored when planes == 1)
    return d


def _run_metadata(pkg, dev, desc, tables2d, count, size, width, page, planes, out_width,
                  out_stride):
    o = dict(slots=torch.full((size,), -7, dtype=torch.int64, device=dev),
             positions=torch.full((size,), -7, dtype=torch.int64, device=dev),
             lengths=torch.full((size,), -7, dtype=torch.int32, device=dev),
             blocks=torch.full((size,), -7, dtype=torch.int64, device=dev),
             offsets=torch.full((size,), -7, dtype=torch.int64, device=dev),
             tables=torch.full((size, out_stride), -7, dtype=torch.int32, device=dev))
    pkg.routing.route_metadata(desc, tables2d, o["slots"], o["positions"], o["lengths"],
                               o["blocks"], o["offsets"], o["tables"], count, size, width, page,
                               planes, out_width)
    return o


def _check_metadata(o, want, count, out_width):
    for key in ("slots", "positions", "lengths"):
        assert torch.equal(o[key].cpu(), want[key]), key
    assert torch.equal(o["blocks"][:count].cpu(), want["blocks"])
    assert torch.equal(o["offsets"][:count].cpu(), want["offsets"])
    assert bool((o["blocks"][count:] == -7).all())  # rows past count: no write address
    assert torch.equal(o["tables"][:, :out_width].cpu(), want["tables"])
    assert bool((o["tables"][:, out_width:] == -7).all())


@pytest.mark.parametrize("planes", [1, 4])
@pytest.mark.parametrize("count,size", [(0, 5), (7, 7), (13, 32)])
def test_route_metadata_matches_oracle(pkg, dev, planes, count, size):
    g = torch.Generator().manual_seed(planes * 100 + count)
    slots, width, page = 6, 300, 16  # width > 256 exercises the column loop
    tables = torch.randint(0, 5000, (slots * planes, width), generator=g, dtype=torch.int32)
    desc = _descriptors(g, count, slots, planes, width, page)
    out_width = width - 3
    o = _run_metadata(pkg, dev, desc.to(dev), tables.to(dev), count, size, width, page, planes,
                      out_width, width + 4)
    want = orr.metadata(desc, tables, count, size, width, page, planes, out_width)
    _check_metadata(o, want, count, out_width)
    s = torch.full((size + 2,), -7, dtype=torch.int64, device=dev)
    pkg.routing.route_slots(desc.to(dev), s, count, size)
    assert torch.equal(s[:size].cpu(), orr.slots(desc, count, size))
    assert bool((s[size:] == -7).all())


@pytest.mark.parametrize("dtype,h", [(torch.bfloat16, 4096), (torch.int64, 1),
                                     (torch.float16, 7), (torch.float32, 33)])
def test_gather_scatter_rows_match_oracle(pkg, dev, dtype, h):
    g = torch.Generator().manual_seed(h)
    rows = 20
    pool = (torch.randn(rows, h, generator=g) * 100).to(dtype)
    ids = torch.randperm(rows, generator=g)[:10]
    ids[4] = rows + 3   # outside the pool
    ids[7] = -1
    out = torch.full((12, h), 5, dtype=dtype, device=dev)
    pkg.routing.gather_rows(pool.to(dev), ids.to(dev), out, 8, 10)
    want = orr.gather_rows(pool, ids, 8, 10)
    assert torch.equal(out[:10].cpu(), want) and bool((out[10:] == 5).all())
    back = torch.zeros(rows, h, dtype=dtype, device=dev)
    pkg.routing.scatter_rows(out[:10], ids.to(dev), back, 8)
    want_back = torch.zeros(rows, h, dtype=dtype)
    orr.scatter_rows(want, ids, want_back, 8)
    assert torch.equal(back.cpu(), want_back)


@pytest.mark.parametrize("dtype,h", [(torch.bfloat16, 2048), (torch.float32, 5)])
def test_segments_match_oracle(pkg, dev, dtype, h):
    g = torch.Generator().manual_seed(9)
    states = torch.randn(6, 40, h, generator=g).to(dtype)
    segs = torch.tensor([[0, 2, 9, 0, 1], [3, 30, 10, 9, 0], [5, 0, 1, 19, 1],
                         [2, 35, 8, 20, 1],    # runs past the slot's rows: clipped
                         [9, 0, 4, 28, 1]])    # slot outside the pool
    out = torch.full((32, h), 3, dtype=dtype, device=dev)
    pkg.routing.gather_segments(states.to(dev), segs.to(dev), out, 10)
    want = torch.full((32, h), 3, dtype=dtype)
    orr.gather_segments(states, segs, want, 10)
    assert torch.equal(out.cpu(), want)
    back = torch.zeros(6, 40, h, dtype=dtype, device=dev)
    pkg.routing.scatter_segments(out, segs.to(dev), back, 10)
    want_back = torch.zeros(6, 40, h, dtype=dtype)
    orr.scatter_segments(want, segs, want_back, 10)
    assert torch.equal(back.cpu(), want_back)


def test_expand_kv_addresses_matches_oracle(pkg, dev):
    g = torch.Generator().manual_seed(11)
    seqs, width, page, n = 9, 40, 16, 300
    tables = torch.randint(0, 10000, (seqs, width), generator=g, dtype=torch.int32)
    pos = torch.randint(0, width * page, (n,), generator=g)
    seq = torch.randint(0, seqs, (n,), generator=g, dtype=torch.int32)
    pos[5], seq[6] = width * page + 1, seqs
    blocks = torch.empty(n, dtype=torch.int64, device=dev)
    offsets = torch.empty_like(blocks)
    pkg.routing.expand_kv_addresses(pos.to(dev), seq.to(dev), tables.to(dev), blocks, offsets,
                                    n, width, page)
    wb, wo = orr.expand_kv_addresses(pos, seq, tables, n, width, page)
    assert torch.equal(blocks.cpu(), wb) and torch.equal(offsets.cpu(), wo)


@pytest.mark.parametrize("with_active", [False, True])
def test_depth_tables_match_reference_formula(pkg, dev, with_active):
    g = torch.Generator().manual_seed(12)
    n, planes, width, page = 40, 4, 64, 16
    wide = torch.randint(0, 9000, (n, planes, width + 8), generator=g, dtype=torch.int32)
    tables = wide[:, :, :width]  # strided view
    depth = torch.randint(0, planes, (n,), generator=g)
    pos = torch.randint(0, width * page, (n,), generator=g)
    active = (torch.rand(n, generator=g) > 0.3) if with_active else None
    tables_d = wide.to(dev)[:, :, :width]
    assert not tables_d.is_contiguous()
    got = pkg.routing.depth_tables(tables_d, depth.to(dev), pos.to(dev), page,
                                   None if active is None else active.to(dev))
    want = orr.depth_tables(tables, depth, pos, page, active)
    for a, b in zip(got, want):
        assert torch.equal(a.cpu(), b)


def test_captured_graph_replays_new_descriptors(pkg, dev):
    """Metadata and the slot gather captured once, replayed with new
    descriptor contents written between replays."""
    g = torch.Generator().manual_seed(13)
    slots, planes, width, page, size, h = 8, 4, 24, 16, 16, 256
    tables = torch.randint(0, 4000, (slots * planes, width), generator=g, dtype=torch.int32)
    hidden = torch.randn(slots, h, generator=g).to(torch.bfloat16)
    tables_d, hidden_d = tables.to(dev), hidden.to(dev)
    desc = torch.zeros(size, 3, dtype=torch.int64, device=dev)
    count = 11
    o = dict(slots=torch.zeros(size, dtype=torch.int64, device=dev),
             positions=torch.zeros(size, dtype=torch.int64, device=dev),
             lengths=torch.zeros(size, dtype=torch.int32, device=dev),
             blocks=torch.zeros(size, dtype=torch.int64, device=dev),
             offsets=torch.zeros(size, dtype=torch.int64, device=dev),
             tables=torch.zeros(size, width, dtype=torch.int32, device=dev))
    gathered = torch.zeros(size, h, dtype=torch.bfloat16, device=dev)

    def body():
        pkg.routing.route_metadata(desc, tables_d, o["slots"], o["positions"], o["lengths"],
                                   o["blocks"], o["offsets"], o["tables"], count, size, width,
                                   page, planes, width)
        pkg.routing.gather_rows(hidden_d, o["slots"], gathered, count, size)

    body()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    for replay in range(3):
        d = _descriptors(g, size, slots, planes, width, page, bad=replay == 2)
        desc.copy_(d.to(dev))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = orr.metadata(d, tables, count, size, width, page, planes, width)
        for key in ("slots", "positions", "lengths", "tables"):
            assert torch.equal(o[key].cpu(), want[key]), (replay, key)
        assert torch.equal(o["blocks"][:count].cpu(), want["blocks"])
        assert torch.equal(gathered.cpu(), orr.gather_rows(hidden, want["slots"], count, size))


def _host_is_device_addressable(t):
    hip = ctypes.CDLL("libamdhip64.so")
    dptr = ctypes.c_void_p()
    rc = hip.hipHostGetDevicePointer(ctypes.byref(dptr), ctypes.c_void_p(t.data_ptr()), 0)
    return rc == 0 and dptr.value == t.data_ptr()


def test_descriptor_in_pinned_host_memory(pkg, dev):
    """The reference stages descriptors in mapped pinned memory (UVA) and launches on
    them directly; the kernels read them through the same pointer."""
    g = torch.Generator().manual_seed(14)
    slots, planes, width, page, count = 5, 2, 12, 16, 9
    host = torch.empty(count, 3, dtype=torch.int64, pin_memory=True)
    if not _host_is_device_addressable(host):
        pytest.skip("pinned host memory is not addressable by the same pointer on this device")
    d = _descriptors(g, count, slots, planes, width, page)
    host.copy_(d)
    tables = torch.randint(0, 900, (slots * planes, width), generator=g, dtype=torch.int32)
    o = _run_metadata(pkg, dev, host, tables.to(dev), count, count, width, page, planes, width,
                      width)
    torch.cuda.synchronize()
    _check_metadata(o, orr.metadata(d, tables, count, count, width, page, planes, width), count,
                    width)
