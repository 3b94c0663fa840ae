"""Device routing and metadata restated on the CPU (test oracle only; the product
never imports this).

* ``slots``            -- vllm_rlt/kernels/routing.py:7-11
* ``metadata``         -- vllm_rlt/kernels/routing.py:14-49
* ``gather_rows`` / ``scatter_rows`` -- routing.py:52-82
* ``gather_segments`` / ``scatter_segments`` -- the host fallbacks of
  vllm_rlt/worker/model_runner.py:544-555 and :585-595 (the device kernels
  routing.py:85-144 are their GPU forms)
* ``expand_kv_addresses`` -- vllm_rlt/kernels/metadata.py:7-24
* ``depth_tables``     -- the tensor formulas of vllm_rlt/worker/async_speculative.py:449-466

Out-of-range indices follow the GPU kernels' contract (the reference would read or
write out of bounds there): gathers read zeros, scatters are skipped, unformable
write blocks are -1.

Pinning: ``depth_tables`` is the reference's own torch formula; ``metadata`` is
checked against ``depth_tables`` (the same addresses through the slot-major plane
tables instead of per-row tables) and ``expand_kv_addresses`` against both;
segment gathers against slicing, row gathers and scatters by round trips.
"""

import torch


def _cmod(a, b):
    """C remainder (sign of the dividend), as the GPU kernels compute it."""
    return a % b if a >= 0 else -((-a) % b)


def slots(descriptor, count, size):
    out = torch.zeros(size, dtype=torch.int64)
    out[:count] = descriptor[:count, 0]
    return out


def metadata(descriptor, tables, count, size, width, page, planes, out_width):
    """tables int32 [slots * planes, width]."""
    rows = tables.shape[0]
    res = dict(slots=torch.zeros(size, dtype=torch.int64),
               positions=torch.zeros(size, dtype=torch.int64),
               lengths=torch.zeros(size, dtype=torch.int32),
               blocks=torch.zeros(count, dtype=torch.int64),
               offsets=torch.zeros(count, dtype=torch.int64),
               tables=torch.zeros(size, out_width, dtype=torch.int32))
    for row in range(count):
        slot, depth, pos = (int(x) for x in descriptor[row])
        plane = depth if planes > 1 else 0
        trow = slot * planes + plane
        table_ok = slot >= 0 and 0 <= plane < planes and trow < rows
        res["slots"][row], res["positions"][row], res["lengths"][row] = slot, pos, pos + 1
        ok = table_ok and pos >= 0 and pos // page < width
        res["blocks"][row] = int(tables[trow, pos // page]) if ok else -1
        res["offsets"][row] = _cmod(pos, page)
        if table_ok:
            res["tables"][row] = tables[trow, :out_width]
    return res


def gather_rows(pool, slot_ids, count, size):
    out = torch.zeros((size,) + tuple(pool.shape[1:]), dtype=pool.dtype)
    for row in range(count):
        s = int(slot_ids[row])
        if 0 <= s < pool.shape[0]:
            out[row] = pool[s]
    return out


def scatter_rows(values, slot_ids, pool, count):
    for row in range(count):
        s = int(slot_ids[row])
        if 0 <= s < pool.shape[0]:
            pool[s] = values[row]


def gather_segments(states, segments, out, max_rows):
    for slot, offset, count, start, _keep in segments.tolist():
        for r in range(min(count, max_rows)):
            if (0 <= slot < states.shape[0] and 0 <= offset + r < states.shape[1]
                    and 0 <= start + r < out.shape[0]):
                out[start + r] = states[slot, offset + r]


def scatter_segments(values, segments, states, max_rows):
    for slot, offset, count, start, keep in segments.tolist():
        if not keep:
            continue
        for r in range(min(count, max_rows)):
            if (0 <= slot < states.shape[0] and 0 <= offset + r < states.shape[1]
                    and 0 <= start + r < values.shape[0]):
                states[slot, offset + r] = values[start + r]


def expand_kv_addresses(positions, sequences, tables, n, width, page):
    tables = tables.reshape(-1, width)
    blocks = torch.empty(n, dtype=torch.int64)
    offsets = torch.empty(n, dtype=torch.int64)
    for i in range(n):
        pos, seq = int(positions[i]), int(sequences[i])
        ok = 0 <= seq < tables.shape[0] and pos >= 0 and pos // page < width
        blocks[i] = int(tables[seq, pos // page]) if ok else -1
        offsets[i] = _cmod(pos, page)
    return blocks, offsets


def depth_tables(tables, depth, positions, block_size, active=None):
    """async_speculative.py:449-466, for in-range depths and positions."""
    table = tables.gather(1, depth[:, None, None].expand(-1, 1, tables.shape[2])).squeeze(1)
    blocks = table.gather(1, (positions // block_size)[:, None]).squeeze(1).long()
    offsets = positions % block_size
    lengths = ((positions + 1) if active is None else torch.where(active, positions + 1, 0)).int()
    return table, blocks, offsets, lengths
