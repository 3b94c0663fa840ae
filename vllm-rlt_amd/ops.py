"""The hot path as torch operators in the ``rlt_mi355x`` namespace.

The reference binds its native code as a ``TORCH_LIBRARY`` schema
(csrc/torch_bindings.cpp:7-13) next to Python ``torch.library`` fragments
(vllm_rlt/kernels/activation.py:34-39).  This package does the same for the gfx950
kernels: the per-step entry points -- ``paged_attention``, ``paged_attention_store``,
``store_kv``, ``spec_probs``, ``categorical``, ``spec_accept``, ``greedy_accept``,
``verify_distributions``, ``verify_accept`` -- are C++ operators
(``csrc/torch_bindings.cpp`` -> ``_C.so``: schema, argument checks, workspace and
launch, one dispatcher call per step); the rest are Python ``torch.library``
custom ops over the same library.  Every operator has an implementation for ROCm
device tensors only (a CPU tensor finds no kernel and raises: there is no
fallback) and a fake (meta) implementation registered here, so that graph capture
and ``torch.compile`` can trace shapes without running them.  The Python shims with
the reference signatures stay in ``attention``, ``sampling`` and ``kv_write``.
"""

from typing import Optional, Tuple

import torch

from . import _lib
from . import kv_write as _kv
from . import sampling as _samp

_lib.ops()  # registers the C++ operators (raises if _C.so is missing)


@torch.library.register_fake("rlt_mi355x::paged_attention")
def _(q, key_cache, value_cache, block_tables, context_lengths, key_scale, value_scale,
      cu_seqlens_q, max_seqlen_q, window, row_lengths=None, compensate=False):
    return torch.empty_like(q)


@torch.library.register_fake("rlt_mi355x::paged_attention_store")
def _(q, k_new, v_new, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q,
      max_seqlen_q, key_scale=None, value_scale=None, row_lengths=None, compensate=False):
    return torch.empty_like(q)


@torch.library.register_fake("rlt_mi355x::spec_probs")
def _(logits, temperature, top_k, top_p, max_top_k, apply_top_p):
    return logits.new_empty(logits.shape, dtype=torch.float32)


@torch.library.register_fake("rlt_mi355x::categorical")
def _(weights, u):
    m = weights.shape[0]
    return (weights.new_empty((m,), dtype=torch.int64), weights.new_empty((m,), dtype=torch.bool))


@torch.library.register_fake("rlt_mi355x::spec_accept")
def _(draft_tokens, drafts, q, p, u_accept, u_final):
    n, w1 = draft_tokens.shape
    i64 = dict(dtype=torch.int64)
    return (p.new_empty((n, w1 + 1), **i64), p.new_empty((n,), **i64), p.new_empty((n,), **i64),
            p.new_empty((n,), dtype=torch.bool))


@torch.library.register_fake("rlt_mi355x::greedy_accept")
def _(draft_tokens, drafts, target_logits):
    n, w1 = draft_tokens.shape
    i64 = dict(dtype=torch.int64)
    return (target_logits.new_empty((n, w1 + 1), **i64), target_logits.new_empty((n,), **i64),
            target_logits.new_empty((n,), **i64))


@torch.library.custom_op("rlt_mi355x::propose_drafts", mutates_args=(), device_types="cuda")
def propose_drafts(logits: torch.Tensor, random_rows: torch.Tensor, temperature: torch.Tensor,
                   top_k: torch.Tensor, top_p: torch.Tensor, u: torch.Tensor, max_top_k: int,
                   apply_top_p: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """(proposed, q_o); reference: vllm_rlt/worker/async_speculative.py:645-663."""
    return _samp.propose_drafts(logits, random_rows, temperature, top_k, top_p, u,
                                max_top_k=max_top_k, apply_top_p=apply_top_p)


@propose_drafts.register_fake
def _(logits, random_rows, temperature, top_k, top_p, u, max_top_k, apply_top_p):
    return (logits.new_empty((logits.shape[0],), dtype=torch.int64),
            logits.new_empty((random_rows.shape[0], logits.shape[1]), dtype=torch.float32))


@torch.library.register_fake("rlt_mi355x::verify_distributions")
def _(logits, random_rows, temperature, top_k, top_p, max_top_k, apply_top_p):
    return (logits.new_empty((logits.shape[0],), dtype=torch.int64),
            logits.new_empty((random_rows.shape[0], logits.shape[1]), dtype=torch.float32))


@torch.library.register_fake("rlt_mi355x::verify_accept")
def _(target_logits, temperature, top_k, top_p, draft_tokens, drafts, q, u_accept, u_final,
      max_top_k, apply_top_p):
    n, w1 = draft_tokens.shape
    i64 = dict(dtype=torch.int64)
    x = target_logits
    return (x.new_empty((n * (w1 + 1),), **i64), x.new_empty(x.shape, dtype=torch.float32),
            x.new_empty((n, w1 + 1), **i64), x.new_empty((n,), **i64), x.new_empty((n,), **i64),
            x.new_empty((n,), dtype=torch.bool))



@torch.library.custom_op("rlt_mi355x::merge_random_round", mutates_args=(), device_types="cuda")
def merge_random_round(target: torch.Tensor, accepted: torch.Tensor, next_tokens: torch.Tensor,
                       starts: torch.Tensor, input_tokens: torch.Tensor, tokens: torch.Tensor,
                       result_accepted: torch.Tensor, result_final: torch.Tensor,
                       result_error: torch.Tensor, random_requests: torch.Tensor,
                       verify_rows: torch.Tensor, verify_ranks: torch.Tensor,
                       verify_offsets: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor,
                                                              torch.Tensor, torch.Tensor,
                                                              torch.Tensor, torch.Tensor]:
    """(rows, accepted, next_tokens, next_positions, next_values, error); reference:
    vllm_rlt/worker/async_speculative.py:162-198."""
    res = _samp.AcceptResult(tokens, result_accepted, result_final, result_error)
    return tuple(_samp.merge_random_round(target, accepted, next_tokens, starts, input_tokens,
                                          res, random_requests, verify_rows, verify_ranks,
                                          verify_offsets))


@merge_random_round.register_fake
def _(target, accepted, next_tokens, starts, input_tokens, tokens, result_accepted, result_final,
      result_error, random_requests, verify_rows, verify_ranks, verify_offsets):
    n = starts.shape[0]
    i64 = dict(dtype=torch.int64)
    return (target.new_empty(target.shape, **i64), starts.new_empty((n,), **i64),
            starts.new_empty((n,), **i64), starts.new_empty((n,), **i64),
            starts.new_empty((n, 2), **i64), starts.new_empty((n,), **i64))

@torch.library.custom_op("rlt_mi355x::rejection_rows", mutates_args=(), device_types="cuda")
def rejection_rows(candidates: torch.Tensor, counts: torch.Tensor, target: torch.Tensor,
                   proposal: torch.Tensor, uniforms: torch.Tensor,
                   sum_threads: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """reference: vllm_rlt/worker/speculative.py:56-72 rejection_sample (device part)."""
    return _samp.rejection_rows(candidates, counts, target, proposal, uniforms,
                                sum_threads=sum_threads)


@rejection_rows.register_fake
def _(candidates, counts, target, proposal, uniforms, sum_threads):
    n = candidates.shape[0]
    return (candidates.new_empty((n,), dtype=torch.int32),
            candidates.new_empty((n,), dtype=torch.int64),
            target.new_empty((n, target.shape[-1]), dtype=torch.float32))


@torch.library.register_fake("rlt_mi355x::store_kv")
def _(key_cache, value_cache, k, v, blocks, offsets, mask, active):
    return None


@torch.library.custom_op("rlt_mi355x::store_fp8",
                         mutates_args=("key_codes", "value_codes", "key_scale", "value_scale"),
                         device_types="cuda")
def store_fp8(k: torch.Tensor, v: torch.Tensor, key_codes: torch.Tensor,
              value_codes: torch.Tensor, key_scale: torch.Tensor, value_scale: torch.Tensor,
              blocks: torch.Tensor, offsets: torch.Tensor, mask: Optional[torch.Tensor],
              active: Optional[torch.Tensor], fixed_scale: Optional[float]) -> None:
    """reference: vllm_rlt/kernels/triton_attention.py:579-623."""
    _kv.store_fp8(k, v, key_codes, value_codes, key_scale, value_scale, blocks, offsets,
                  _kv.FP8_E4M3_MAX, mask=mask, active=active, fixed_scale=fixed_scale)


@torch.library.custom_op("rlt_mi355x::finalize_rows", mutates_args=("key_pool", "value_pool"),
                         device_types="cuda")
def finalize_rows(descriptor: torch.Tensor, tables: torch.Tensor, key_pool: torch.Tensor,
                  value_pool: torch.Tensor, block_size: int) -> None:
    """reference: vllm_rlt/kernels/routing.py:147-180 finalize_kernel."""
    _kv.finalize_rows(descriptor, tables, key_pool, value_pool, block_size)


OPS = ("paged_attention", "paged_attention_store", "spec_probs", "categorical", "spec_accept", "greedy_accept",
       "propose_drafts", "verify_distributions", "verify_accept", "merge_random_round",
       "rejection_rows", "store_kv",
       "store_fp8", "finalize_rows")
