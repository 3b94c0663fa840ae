"""KV write side restated (test oracle only; nothing in the product imports this).

* ``store_kv``      -- the index-put writer: row i of k/v lands at
  (blocks[i], offsets[i]) of one layer's [block, token, kv_head, dim] view
  (vllm_rlt/core/kv_cache_manager.py:893-895), with the device-masked forms'
  row skipping: ``mask`` false or row >= ``active`` (vllm_rlt/kernels/routing.py:
  210-223 masked_kv_store, vllm_rlt/kernels/graph_kv.py:52-67 write_graph_kv).
* ``store_fp8``     -- the same scatter of ``quantize_fp8`` codes and scales
  (vllm_rlt/kernels/triton_attention.py:579-623, bitwise equal to
  vllm_rlt/core/kv_cache_manager.py:50-61).
* ``finalize_rows`` -- the LAST_EXITED copy, host form of
  vllm_rlt/kernels/routing.py:147-180 following vllm_rlt/core/kv_cache_manager.py:
  1053-1076 finalize_token: for each (slot, exit depth, position), every layer's
  entry at the position's page offset is copied from the exit plane's block into
  the blocks of all deeper planes.
* ``e4m3_encode``   -- an independent e4m3fn encoder built from the format's
  definition (bias 7, 3 mantissa bits, subnormal step 2^-9, maximum 448, code
  0x7f/0xff = NaN, no infinities): the nearest representable value, ties to the
  even code.  It pins torch's ``float8_e4m3fn`` cast that ``quantize_fp8`` uses.

Rows or descriptors addressing memory outside the pool are skipped, as the GPU
kernels do (the reference's kernels would write out of bounds there).

Pinning: ``e4m3_encode`` == torch's cast on every float16 value and on random
float32 values; ``store_fp8`` meets the reference's known-answer tests
(tests/test_fp8_kv_cache.py:46-55 per-vector bound amax/16 and zero vectors,
tests/test_fa4_fp8.py:39-49 saturation under a fixed scale); ``finalize_rows``
against the reference's finalize test (tests/test_fp8_kv_cache.py:142-152) and a
per-element brute force.
"""

import numpy as np
import torch

from .fp8 import quantize_fp8


def _e4m3_table():
    values = np.zeros(128, dtype=np.float64)
    for code in range(128):
        e, m = code >> 3, code & 7
        values[code] = m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
    values[0x7F] = np.nan
    return values


_E4M3 = _e4m3_table()


def e4m3_encode(x):
    """float32 array (|x| <= 448 or NaN) -> uint8 e4m3fn codes."""
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    a = np.abs(x).ravel()
    finite = _E4M3[:0x7F]
    idx = np.searchsorted(finite, a)                 # finite[idx-1] < a <= finite[idx]
    hi = np.clip(idx, 0, 0x7E)
    lo = np.clip(idx - 1, 0, 0x7E)
    d_hi, d_lo = finite[hi] - a, a - finite[lo]
    pick = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, hi, np.where(lo % 2 == 0, lo, hi)))
    code = pick.astype(np.uint8)
    code[np.isnan(a)] = 0x7F
    sign = (np.signbit(x.ravel())).astype(np.uint8) << 7
    return (code | sign).reshape(x.shape)


def _keep(rows, blocks, offsets, mask, active, num_blocks, block_size):
    keep = np.ones(rows, dtype=bool)
    if mask is not None:
        keep &= mask.cpu().numpy().astype(bool)
    if active is not None:
        keep &= np.arange(rows) < int(active)
    b, o = blocks.cpu().numpy(), offsets.cpu().numpy()
    keep &= (b >= 0) & (b < num_blocks) & (o >= 0) & (o < block_size)
    return np.nonzero(keep)[0]


def store_kv(key_cache, value_cache, k, v, blocks, offsets, mask=None, active=None):
    rows = k.shape[0]
    idx = _keep(rows, blocks, offsets, mask, active, key_cache.shape[0], key_cache.shape[1])
    for i in idx:
        b, o = int(blocks[i]), int(offsets[i])
        key_cache[b, o] = k[i]
        value_cache[b, o] = v[i]


def store_fp8(k, v, key_codes, value_codes, key_scale, value_scale, blocks, offsets,
              mask=None, active=None, fixed_scale=None):
    rows = k.shape[0]
    idx = _keep(rows, blocks, offsets, mask, active, key_codes.shape[0], key_codes.shape[1])
    for x, codes, scales in ((k, key_codes, key_scale), (v, value_codes, value_scale)):
        c, s = quantize_fp8(x, fixed_scale)
        for i in idx:
            b, o = int(blocks[i]), int(offsets[i])
            codes[b, o] = c[i]
            scales[b, o] = s[i]


def finalize_rows(descriptor, tables, key_pool, value_pool, block_size):
    """descriptor [rows, 3] = (slot, depth, position); tables [slots, planes, width];
    pools [block, layer, token, ...]."""
    slots, planes, width = tables.shape
    nblocks = key_pool.shape[0]
    for slot, depth, pos in descriptor.tolist():
        if not (0 <= slot < slots and 0 <= depth and 0 <= pos < width * block_size):
            continue
        page, off = divmod(pos, block_size)
        src = int(tables[slot, depth, page]) if depth < planes else -1
        if not 0 <= src < nblocks:
            continue
        for target in range(depth + 1, planes):
            dst = int(tables[slot, target, page])
            if 0 <= dst < nblocks:
                key_pool[dst, :, off] = key_pool[src, :, off]
                value_pool[dst, :, off] = value_pool[src, :, off]
