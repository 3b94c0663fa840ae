"""MI355X KV write side behind the reference's writer functions.

Same arguments and semantics as
* vllm_rlt/kernels/routing.py:210-223 ``masked_kv_store(keys, values, k, v, metadata)``,
* vllm_rlt/kernels/graph_kv.py:52-67 ``write_graph_kv(key_cache, value_cache, batch, k, v)``,
* vllm_rlt/kernels/triton_attention.py:579-623 ``store_fp8(k, v, key_codes, value_codes,
  key_scale, value_scale, blocks, offsets, fp8_max, *, mask=None, active=None,
  fixed_scale=None)`` (bitwise equal to kv_cache_manager.quantize_fp8),
* vllm_rlt/kernels/routing.py:147-180 ``finalize_kernel`` (``finalize_rows`` here, the
  LAST_EXITED copy into deeper planes),
plus ``store_kv``, the unmasked index-put writer
(vllm_rlt/core/kv_cache_manager.py:893-895).  Every call enqueues one gfx950 launch on
the current stream without host synchronization.  Rows whose block or offset lies
outside the pool are skipped (the reference's kernels would write out of bounds).
"""

import torch

from . import _lib

FP8_E4M3_MAX = 448.0
_ROW_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _rows(x, name):
    if x.ndim != 3:
        raise ValueError(f"{name} must be [rows, kv_heads, head_dim]")
    return x if x.stride(-1) == 1 else x.contiguous()


def _index(t, rows, name):
    if t.shape != (rows,):
        raise ValueError(f"{name} must have shape [{rows}]")
    t = t if t.dtype == torch.int64 else t.long()
    return t if t.is_contiguous() else t.contiguous()


def _mask(mask, rows):
    if mask is None:
        return None
    if mask.shape != (rows,):
        raise ValueError(f"mask must have shape [{rows}]")
    m = mask if mask.dtype in (torch.bool, torch.uint8) else mask.bool()
    return m.contiguous()


def _active(active):
    if active is None:
        return None
    if active.numel() != 1:
        raise ValueError("active must be one int32 row count")
    return active.reshape(()).to(torch.int32).contiguous()


def _check_view(cache, name):
    if cache.ndim != 4 or cache.stride(-1) != 1:
        raise ValueError(f"{name} must be a [block, token, kv_head, dim] view with unit dim stride")


def store_kv(key_cache, value_cache, k, v, blocks, offsets, *, mask=None, active=None):
    """Scatter rows k, v [rows, kv_heads, head_dim] into one layer's pool views
    [block, token, kv_head, dim] at (blocks[i], offsets[i]); rows with a false
    ``mask`` entry or at/after ``*active`` are skipped."""
    _check_view(key_cache, "key_cache")
    _check_view(value_cache, "value_cache")
    if key_cache.stride() != value_cache.stride() or key_cache.shape != value_cache.shape:
        raise ValueError("key and value pools must share a layout")
    k, v = _rows(k, "k"), _rows(v, "v")
    rows = k.shape[0]
    if v.shape != k.shape or k.shape[1:] != key_cache.shape[2:]:
        raise ValueError("k, v must be [rows, kv_heads, head_dim] of the pool")
    if k.dtype != key_cache.dtype or v.dtype != key_cache.dtype:
        raise ValueError("rows must have the pool's dtype")
    _lib.require_gpu(key_cache, value_cache, k, v, blocks, offsets, mask, active)
    if rows == 0:
        return
    # the operator reads int64 indices, a bool / uint8 mask and an int32 count as given
    # (it raises on anything else): torch.ops.rlt_mi355x.store_kv
    _lib.ops().store_kv(key_cache, value_cache, k, v, _index(blocks, rows, "blocks"),
                        _index(offsets, rows, "offsets"), _mask(mask, rows), _active(active))


def masked_kv_store(keys, values, k, v, metadata):
    """reference: vllm_rlt/kernels/routing.py:210-223 (rows with a false
    ``metadata.write_mask`` entry are skipped)."""
    store_kv(keys, values, k, v, metadata.write_blocks, metadata.write_offsets,
             mask=metadata.write_mask)


def write_graph_kv(key_cache, value_cache, batch, k, v):
    """reference: vllm_rlt/kernels/graph_kv.py:52-67 (``batch.active_rows`` and
    ``batch.write_mask`` skip rows on the device)."""
    store_kv(key_cache, value_cache, k, v, batch.write_blocks, batch.write_offsets,
             mask=getattr(batch, "write_mask", None), active=getattr(batch, "active_rows", None))


def store_fp8(k, v, key_codes, value_codes, key_scale, value_scale, blocks, offsets, fp8_max,
              *, mask=None, active=None, fixed_scale=None):
    """Quantize rows k, v [row, KV head, dim] and scatter codes and scales in one launch.

    reference: vllm_rlt/kernels/triton_attention.py:579-623.  Codes and scales are
    bitwise those of ``quantize_fp8`` (vllm_rlt/core/kv_cache_manager.py:50-61).
    """
    if k.shape[0] == 0:
        return
    if fp8_max != FP8_E4M3_MAX:
        raise ValueError("fp8_max must be 448 (OCP e4m3fn)")
    if key_codes.stride() != value_codes.stride() or key_scale.stride() != value_scale.stride():
        raise ValueError("FP8 key and value pools must share a layout")
    _check_view(key_codes, "key_codes")
    if key_codes.dtype != torch.float8_e4m3fn or value_codes.dtype != torch.float8_e4m3fn:
        raise ValueError("code pools must be float8_e4m3fn")
    if key_scale.ndim != 3 or key_scale.dtype != torch.float32:
        raise ValueError("scale pools must be float32 [block, token, kv_head]")
    k, v = _rows(k, "k"), _rows(v, "v")
    if k.dtype not in _ROW_DTYPES or v.dtype != k.dtype:
        raise ValueError("k and v must share a float dtype")
    rows = k.shape[0]
    if v.shape != k.shape or k.shape[1:] != key_codes.shape[2:]:
        raise ValueError("k, v must be [rows, kv_heads, head_dim] of the pool")
    _lib.require_gpu(k, v, key_codes, value_codes, key_scale, value_scale, blocks, offsets,
                     mask, active)
    b, o = _index(blocks, rows, "blocks"), _index(offsets, rows, "offsets")
    m, a = _mask(mask, rows), _active(active)
    lib = _lib.library()
    status = lib.rlt_kv_store_fp8(
        _lib.ptr(k), _lib.ptr(v), _lib.dtype_code(k.dtype), k.stride(0), k.stride(1),
        v.stride(0), v.stride(1), _lib.ptr(key_codes), _lib.ptr(value_codes),
        key_codes.stride(0), key_codes.stride(1), key_codes.stride(2), _lib.ptr(key_scale),
        _lib.ptr(value_scale), key_scale.stride(0), key_scale.stride(1), key_scale.stride(2),
        key_codes.shape[0], key_codes.shape[1], _lib.ptr(b), _lib.ptr(o), _lib.ptr(m),
        _lib.ptr(a), rows, k.shape[1], k.shape[2], int(fixed_scale is not None),
        float(fixed_scale) if fixed_scale is not None else 0.0, _lib.stream_of(k.device))
    _lib.check(status, "rlt_kv_store_fp8")


def finalize_rows(descriptor, tables, key_pool, value_pool, block_size):
    """LAST_EXITED copy: for each descriptor row (slot, exit depth, position), every
    layer's K/V at the position's page offset is copied from the exit plane's block
    into the same offset of every deeper plane's block.

    reference: vllm_rlt/kernels/routing.py:147-180 (finalize_kernel, launched per
    pool pair at vllm_rlt/worker/model_runner.py:1356-1390).  ``tables`` int32
    [slots, planes, width]; pools [block, layer, token, ...] (code / value pools, or
    the fp32 scale pools of an FP8 cache).
    """
    if descriptor.ndim != 2 or descriptor.shape[-1] != 3:
        raise ValueError("descriptor must be [rows, 3] = (slot, depth, position)")
    if tables.ndim != 3:
        raise ValueError("tables must be [slots, planes, width]")
    if key_pool.shape != value_pool.shape or key_pool.stride() != value_pool.stride():
        raise ValueError("key and value pools must share a layout")
    if key_pool.ndim < 3 or key_pool.dtype != value_pool.dtype:
        raise ValueError("pools must be [block, layer, token, ...] of one dtype")
    _lib.require_gpu(descriptor, tables, key_pool, value_pool)
    rows = descriptor.shape[0]
    if rows == 0:
        return
    d = descriptor.to(torch.int64).contiguous()
    tb = tables.to(torch.int32).contiguous()
    tail = key_pool[0, 0, 0]
    per_token = tail.numel() * key_pool.element_size()
    if not tail.is_contiguous():
        raise ValueError("the per-token channels of the pools must be contiguous")
    lib = _lib.library()
    status = lib.rlt_kv_finalize(
        _lib.ptr(d), rows, _lib.ptr(tb), tb.shape[0], tb.shape[2], tb.shape[1], block_size,
        key_pool.shape[1], key_pool.shape[0], _lib.ptr(key_pool), _lib.ptr(value_pool),
        key_pool.stride(0), key_pool.stride(1), key_pool.stride(2), per_token,
        key_pool.element_size(), _lib.stream_of(key_pool.device))
    _lib.check(status, "rlt_kv_finalize")
