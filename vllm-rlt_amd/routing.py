"""MI355X device routing and metadata for the asynchronous verify step.

Each function replaces one Triton launch of the reference with the same buffers and
meaning; grids depend only on the capacities given, so the calls are capturable in
HIP graphs and replay with new descriptor contents:

* ``route_slots``        -- vllm_rlt/kernels/routing.py:7-11 ``slots_kernel``
* ``route_metadata``     -- routing.py:14-49 ``metadata_kernel``
  (caller vllm_rlt/worker/async_state.py:65-97 ``materialize_metadata``)
* ``gather_rows`` / ``scatter_rows`` -- routing.py:52-82 ``gather_kernel`` /
  ``scatter_kernel`` (async_state.py:104-123, async_speculative.py:605-615,754-760)
* ``gather_segments`` / ``scatter_segments`` -- routing.py:85-144
  (vllm_rlt/worker/model_runner.py:519-584)
* ``expand_kv_addresses`` -- vllm_rlt/kernels/metadata.py:7-24
  (vllm_rlt/worker/buffers.py:289-335)
* ``depth_tables``       -- the per-row plane-table gather, write address and context
  lengths of vllm_rlt/worker/async_speculative.py:449-466 in one launch.

Indices read from memory are bounds-checked on the device: a gather from outside
its pool yields zeros, a scatter outside its pool is skipped, and a write block that
cannot be formed is -1 (skipped by the KV writers).
"""

import torch

from . import _lib


def _dev(*tensors):
    _lib.require_gpu(*tensors)


def _check(t, name, dtype, ndim=None):
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}")
    if ndim is not None and t.ndim != ndim:
        raise ValueError(f"{name} must have {ndim} dimensions")


def _rows2d(t, name):
    if t.ndim == 1:
        t = t.view(-1, 1)
    if t.ndim != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a [rows, elements] view with unit element stride")
    return t


def _descriptor(d, name="descriptor"):
    """A device tensor or, as the reference stages them, pinned (mapped) host memory."""
    _check(d, name, torch.int64)
    if d.ndim != 2 or d.shape[1] != 3 or not d.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int64 [rows, 3]")
    if d.device.type != "cuda" and not d.is_pinned():
        raise ValueError(f"{name} must be a ROCm device tensor or pinned host memory")
    return d


def route_slots(descriptor, slots, count, size=None):
    """slots[:count] = descriptor[:count, 0]; slots[count:size] = 0."""
    size = slots.shape[0] if size is None else size
    _check(slots, "slots", torch.int64, 1)
    if count > 0:
        _descriptor(descriptor)
        if descriptor.shape[0] < count:
            raise ValueError("descriptor has fewer rows than count")
    if not 0 <= count <= size <= slots.shape[0]:
        raise ValueError("need 0 <= count <= size <= len(slots)")
    _dev(slots)
    _lib.check(_lib.library().rlt_route_slots(_lib.ptr(descriptor if count > 0 else None),
                                              _lib.ptr(slots), count, size,
                                              _lib.stream_of(slots.device)), "rlt_route_slots")


def route_metadata(descriptor, tables, slots, positions, lengths, blocks, offsets, out_tables,
                   count, size, width, page, planes, out_width):
    """Per-row metadata from (slot, depth, position) descriptors; ``tables`` int32
    [slots * planes, width] slot-major (the reference's ``owner.tables`` viewed 2-D)."""
    tables = tables.reshape(-1, width)
    _check(tables, "tables", torch.int32)
    for t, name, dt in ((slots, "slots", torch.int64), (positions, "positions", torch.int64),
                        (lengths, "lengths", torch.int32), (blocks, "blocks", torch.int64),
                        (offsets, "offsets", torch.int64)):
        _check(t, name, dt, 1)
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    _check(out_tables, "out_tables", torch.int32, 2)
    if out_tables.stride(1) != 1 or not tables.is_contiguous():
        raise ValueError("tables must be row-major with unit column stride")
    if not 0 <= count <= size or size > min(len(slots), len(positions), len(lengths),
                                            out_tables.shape[0]):
        raise ValueError("need 0 <= count <= size <= the output capacities")
    if count > min(len(blocks), len(offsets)) or out_width > out_tables.shape[1]:
        raise ValueError("blocks / offsets / out_tables too small")
    if count > 0:
        _descriptor(descriptor)
        if descriptor.shape[0] < count:
            raise ValueError("descriptor has fewer rows than count")
    _dev(tables, slots, positions, lengths, blocks, offsets,
         out_tables)
    status = _lib.library().rlt_route_metadata(
        _lib.ptr(descriptor if count > 0 else None), _lib.ptr(tables), tables.shape[0], width,
        page, planes, _lib.ptr(slots), _lib.ptr(positions), _lib.ptr(lengths), _lib.ptr(blocks),
        _lib.ptr(offsets), _lib.ptr(out_tables), out_tables.stride(0), out_width, count, size,
        _lib.stream_of(slots.device))
    _lib.check(status, "rlt_route_metadata")


def gather_rows(pool, slots, out, count, size=None):
    """out[row] = pool[slots[row]] for row < count, zeros for count <= row < size."""
    pool, out = _rows2d(pool, "pool"), _rows2d(out, "out")
    size = out.shape[0] if size is None else size
    if pool.dtype != out.dtype or pool.shape[1] != out.shape[1]:
        raise ValueError("pool and out must share dtype and row width")
    _check(slots, "slots", torch.int64, 1)
    if not 0 <= count <= size <= out.shape[0] or count > slots.shape[0]:
        raise ValueError("need 0 <= count <= size <= len(out), count <= len(slots)")
    if not slots.is_contiguous():
        raise ValueError("slots must be contiguous")
    _dev(pool, slots, out)
    status = _lib.library().rlt_route_gather(
        _lib.ptr(pool), pool.shape[0], pool.stride(0), _lib.ptr(slots), _lib.ptr(out),
        out.stride(0), count, size, out.shape[1], out.element_size(), _lib.stream_of(out.device))
    _lib.check(status, "rlt_route_gather")


def scatter_rows(values, slots, pool, count=None):
    """pool[slots[row]] = values[row] for row < count."""
    values, pool = _rows2d(values, "values"), _rows2d(pool, "pool")
    count = values.shape[0] if count is None else count
    if pool.dtype != values.dtype or pool.shape[1] != values.shape[1]:
        raise ValueError("values and pool must share dtype and row width")
    _check(slots, "slots", torch.int64, 1)
    if not 0 <= count <= min(values.shape[0], slots.shape[0]):
        raise ValueError("count exceeds values or slots")
    if not slots.is_contiguous():
        raise ValueError("slots must be contiguous")
    _dev(values, slots, pool)
    status = _lib.library().rlt_route_scatter(
        _lib.ptr(values), values.stride(0), _lib.ptr(slots), _lib.ptr(pool), pool.shape[0],
        pool.stride(0), count, pool.shape[1], pool.element_size(), _lib.stream_of(pool.device))
    _lib.check(status, "rlt_route_scatter")


def _segments(segments):
    _check(segments, "segments", torch.int64, 2)
    if segments.shape[1] != 5 or not segments.is_contiguous():
        raise ValueError("segments must be a contiguous int64 [segments, 5]")
    return segments


def gather_segments(states, segments, out, max_rows):
    """``states`` [slots, rows_per_slot, h]: out[start + r] = states[slot, offset + r]
    for r < count (segments int64 [S, 5] = slot, offset, count, start, keep)."""
    if states.ndim != 3 or not states.is_contiguous():
        raise ValueError("states must be a contiguous [slots, rows_per_slot, h] pool")
    out = _rows2d(out, "out")
    if out.dtype != states.dtype or out.shape[1] != states.shape[2]:
        raise ValueError("states and out must share dtype and row width")
    _segments(segments)
    _dev(states, segments, out)
    status = _lib.library().rlt_route_gather_segments(
        _lib.ptr(states), states.shape[0], states.shape[1], states.shape[2], _lib.ptr(segments),
        segments.shape[0], max_rows, _lib.ptr(out), out.shape[0], out.stride(0), out.shape[1],
        out.element_size(), _lib.stream_of(out.device))
    _lib.check(status, "rlt_route_gather_segments")


def scatter_segments(values, segments, states, max_rows):
    """Kept segments only: states[slot, offset + r] = values[start + r] for r < count."""
    if states.ndim != 3 or not states.is_contiguous():
        raise ValueError("states must be a contiguous [slots, rows_per_slot, h] pool")
    values = _rows2d(values, "values")
    if values.dtype != states.dtype or values.shape[1] != states.shape[2]:
        raise ValueError("values and states must share dtype and row width")
    _segments(segments)
    _dev(values, segments, states)
    status = _lib.library().rlt_route_scatter_segments(
        _lib.ptr(values), values.shape[0], values.stride(0), _lib.ptr(segments),
        segments.shape[0], max_rows, _lib.ptr(states), states.shape[0], states.shape[1],
        states.shape[2], values.shape[1], values.element_size(), _lib.stream_of(values.device))
    _lib.check(status, "rlt_route_scatter_segments")


def expand_kv_addresses(positions, sequences, tables, blocks, offsets, n, width, page):
    """blocks[i] = tables[sequences[i], positions[i] // page], offsets[i] = positions[i] % page."""
    _check(positions, "positions", torch.int64, 1)
    _check(sequences, "sequences", torch.int32, 1)
    _check(tables, "tables", torch.int32)
    _check(blocks, "blocks", torch.int64, 1)
    _check(offsets, "offsets", torch.int64, 1)
    tables = tables.reshape(-1, width)
    if not tables.is_contiguous() or not all(t.is_contiguous() for t in
                                             (positions, sequences, blocks, offsets)):
        raise ValueError("inputs must be contiguous")
    if n > min(len(positions), len(sequences), len(blocks), len(offsets)):
        raise ValueError("n exceeds a buffer")
    _dev(positions, sequences, tables, blocks, offsets)
    status = _lib.library().rlt_expand_kv_addresses(
        _lib.ptr(positions), _lib.ptr(sequences), _lib.ptr(tables), tables.shape[0], width, page,
        _lib.ptr(blocks), _lib.ptr(offsets), n, _lib.stream_of(blocks.device))
    _lib.check(status, "rlt_expand_kv_addresses")


def depth_tables(tables, depth, positions, block_size, active=None):
    """(table int32 [n, width], write_blocks int64 [n], write_offsets int64 [n],
    context_lengths int32 [n]) for rows at plane ``depth[row]`` of ``tables`` int32
    [n, planes, width]; lengths are 0 where ``active`` is false."""
    _check(tables, "tables", torch.int32, 3)
    _check(depth, "depth", torch.int64, 1)
    _check(positions, "positions", torch.int64, 1)
    n, planes, width = tables.shape
    if tables.stride(2) != 1:
        raise ValueError("tables must have unit column stride")
    if depth.shape[0] != n or positions.shape[0] != n:
        raise ValueError("depth and positions must have one entry per row")
    if active is not None:
        if active.shape != (n,):
            raise ValueError("active must be [n]")
        active = (active if active.dtype in (torch.bool, torch.uint8) else active.bool()).contiguous()
    depth, positions = depth.contiguous(), positions.contiguous()
    _dev(tables, depth, positions, active)
    dev = tables.device
    table = torch.empty(n, width, dtype=torch.int32, device=dev)
    blocks = torch.empty(n, dtype=torch.int64, device=dev)
    offsets = torch.empty(n, dtype=torch.int64, device=dev)
    lengths = torch.empty(n, dtype=torch.int32, device=dev)
    status = _lib.library().rlt_depth_tables(
        _lib.ptr(tables), tables.stride(0), tables.stride(1), planes, width, _lib.ptr(depth),
        _lib.ptr(positions), _lib.ptr(active), block_size, _lib.ptr(table), table.stride(0),
        _lib.ptr(blocks), _lib.ptr(offsets), _lib.ptr(lengths), n, _lib.stream_of(dev))
    _lib.check(status, "rlt_depth_tables")
    return table, blocks, offsets, lengths
