"""Torch-CPU restatement of the reference paged attention (test oracle only).

Follows vllm_rlt/kernels/paged_attention.py:13-47 (``torch_paged_attention``)
and :50-90 (``torch_paged_attention_windowed``) operation for operation: a
Python loop over rows, fancy-index gathers of the row's keys and values in
fp32, optional per-vector FP8 scales multiplied in fp32, GQA by
``repeat_interleave``, fp32 ``softmax(q k^T / sqrt(D)) v``, cast to q's dtype,
and a zero row for length 0.

The packed verify-window form (``packed_window_attention``) expands each
sequence into per-row lengths exactly as the reference test does
(tests/test_attention.py:134-147 with the bottom-right alignment of
vllm_rlt/kernels/triton_attention.py:396-401): query ``i`` of a sequence with
``q_len`` rows and ``kv_len`` keys sees keys ``< kv_len - q_len + i + 1``.
"""

import math

import torch


def _scale_rows(scale, blocks, offsets):
    # A 0-d scale is the fixed per-tensor FP8 scale; the reference oracle
    # stores it as a per-vector pool filled with the constant
    # (vllm_rlt/core/kv_cache_manager.py:267-271), which multiplies identically.
    if scale.dim() == 0:
        return scale.expand(blocks.shape[0], 1)
    return scale[blocks, offsets]


def paged_attention(q, key_cache, value_cache, block_tables, context_lengths,
                    key_scale=None, value_scale=None, window=0):
    """Per-row paged attention; ``window > 0`` keeps only the last ``window`` keys.

    reference: vllm_rlt/kernels/paged_attention.py:13-47 (window == 0) and
    :50-90 (window > 0).
    """
    output = torch.empty_like(q)
    block_size = key_cache.shape[1]
    head_groups = q.shape[1] // key_cache.shape[2]
    scale = 1.0 / math.sqrt(q.shape[-1])
    for row, length in enumerate(context_lengths.tolist()):
        if length == 0:
            output[row].zero_()
            continue
        first = max(0, length - window) if window else 0
        token_positions = torch.arange(first, length, device=q.device)
        blocks = block_tables[row, token_positions // block_size].long()
        offsets = token_positions % block_size
        keys = key_cache[blocks, offsets].float()
        values = value_cache[blocks, offsets].float()
        if key_scale is not None:
            keys = keys * _scale_rows(key_scale, blocks, offsets).unsqueeze(-1)
            values = values * _scale_rows(value_scale, blocks, offsets).unsqueeze(-1)
        keys = keys.repeat_interleave(head_groups, dim=1)
        values = values.repeat_interleave(head_groups, dim=1)
        scores = torch.einsum("hd,thd->ht", q[row].float(), keys.float()) * scale
        probabilities = torch.softmax(scores, dim=-1)
        output[row] = torch.einsum("ht,thd->hd", probabilities, values.float()).to(q.dtype)
    return output


def packed_row_layout(context_lengths, cu_seqlens_q):
    """(row -> sequence, row length) of the packed verify window.

    reference: vllm_rlt/kernels/triton_attention.py:396-401 (query i of a
    sequence sits at ``context_length - query_length + i``).
    """
    cu = [int(c) for c in cu_seqlens_q.tolist()]
    lengths = [int(n) for n in context_lengths.tolist()]
    seq_of_row, row_lengths = [], []
    for s, kv_len in enumerate(lengths):
        q_len = cu[s + 1] - cu[s]
        for i in range(q_len):
            seq_of_row.append(s)
            row_lengths.append(kv_len - q_len + i + 1)
    return seq_of_row, row_lengths


def packed_window_attention(q, key_cache, value_cache, block_tables, context_lengths,
                            cu_seqlens_q, key_scale=None, value_scale=None, window=0):
    """Packed causal window through the per-row oracle (one table per sequence)."""
    seq_of_row, row_lengths = packed_row_layout(context_lengths, cu_seqlens_q)
    if not seq_of_row:
        return torch.empty_like(q)
    tables = block_tables[torch.tensor(seq_of_row, dtype=torch.long)]
    lengths = torch.tensor(row_lengths, dtype=torch.int32)
    return paged_attention(q, key_cache, value_cache, tables, lengths,
                           key_scale, value_scale, window)


def dense_attention(q, k, v):
    """Independent closed-form oracle: fp32 SDPA over one row's gathered keys.

    q [Hq, D], k/v [T, Hkv, D]; reference: tests/test_attention.py:8-15.
    """
    groups = q.shape[0] // k.shape[1]
    return torch.nn.functional.scaled_dot_product_attention(
        q.float()[None, :, None],
        k.float().repeat_interleave(groups, dim=1).transpose(0, 1)[None],
        v.float().repeat_interleave(groups, dim=1).transpose(0, 1)[None],
    )[0, :, 0]
