"""CPU oracle for the speculative-verification hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports, links or
calls anything here; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker or the
timed CPU baseline.

Contents (each function cites the reference file:line it restates):

* ``attention``  -- ``torch_paged_attention`` / windowed / packed-window
  semantics (vllm_rlt/kernels/paged_attention.py:13-90,
  vllm_rlt/kernels/triton_attention.py:386-404 for the packed form).
* ``sampling``   -- ``batched_probabilities``, ``Sampler.probabilities``,
  ``categorical``, ``speculative_accept``, greedy prefix accept, the
  synchronous runner's ``rejection_sample`` / random-request round, the
  per-request uniform protocol and the random-round merge
  (vllm_rlt/worker/speculative_sampling.py, worker/sampler.py:28-62,
  worker/speculative.py:41-72, worker/async_speculative.py:101-198,567-586,
  694-770).
* ``fp8``        -- ``quantize_fp8`` / ``dequantize_fp8``
  (vllm_rlt/core/kv_cache_manager.py:40-65).
* ``order``      -- ctypes binding of ``order.c``, an independent C model of
  the two torch-CPU summation orders the acceptance contract depends on:
  the fp32 ``Tensor.sum(-1)`` cascade (and a whole 1-D tensor's ``sum()`` over
  thread chunks) and the sequential fp64 ``cumsum`` feeding ``searchsorted``.  Tests pin it bit-for-bit against torch itself.

Pinning (what fixes each function beyond restating it):

* attention: dense SDPA closed form on gathered keys (``F.scaled_dot_product_
  attention``), single-key rows (output == V), zero-length rows, GQA head
  mapping, FP8 == attention over dequantized values.
* categorical / speculative_accept: every known-answer test of
  tests/test_speculative_sampling.py:170-576 in the reference, exact
  quadrature identities (P(accept) = sum min(p, q), first-token marginal = p0),
  and the C order model.
* batched_probabilities: closed-form KATs (tests/test_speculative.py:474-490),
  top-k tie counts, top_p == 1 softmax identity.
* greedy accept: reference KAT tests/test_speculative.py:277-285 and brute
  force over tiny vocabularies.
* rejection_sample / collect_stochastic: the reference's recovery test
  (tests/test_speculative.py:455-471: the accepted-or-resampled token follows p)
  on CPU generators, exact residual closed forms, the error cases, and the C
  model of the 1-D sum order.
"""
