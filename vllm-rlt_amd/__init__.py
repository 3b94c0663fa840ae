"""vllm_rlt_amd -- MI355X-native speculative-verification hot path of vllm-rlt.

Drop-in host layer over ``librlt_mi355x.so`` (hand-written gfx950 HIP kernels):

* ``attention``: ``BackendCapabilities`` / ``AttentionBackend`` / ``create_backend``
  and the ``MI355XPagedAttention`` kernel object with the reference's per-row
  ``__call__``, ``windowed`` and packed ``prefill`` signatures
  (vllm_rlt/attention/backend.py, vllm_rlt/kernels/paged_attention.py).
* ``sampling``: ``batched_probabilities``, ``categorical``, ``speculative_accept`` /
  ``AcceptResult``, ``greedy_accept`` and the device greedy round
  ``greedy_accept_batched`` (vllm_rlt/worker/speculative_sampling.py,
  vllm_rlt/worker/speculative.py:41-53, vllm_rlt/worker/async_speculative.py:706-720),
  and the synchronous runner's ``rejection_sample`` / ``rejection_round``
  (vllm_rlt/worker/speculative.py:56-72,574-625).
* ``kv_write``: ``store_kv``, ``masked_kv_store``, ``write_graph_kv``, ``store_fp8`` and
  ``finalize_rows``, the KV writers the verify window's keys and values go through
  (vllm_rlt/kernels/routing.py:147-223, vllm_rlt/kernels/graph_kv.py:52-67,
  vllm_rlt/kernels/triton_attention.py:579-623).
* ``ops``: the same entry points as ``torch.ops.rlt_mi355x.*`` operators (ROCm device
  implementations and fake shape functions; the reference's torch_bindings pattern).
* ``routing``: device metadata and request routing of the asynchronous verify step
  (vllm_rlt/kernels/routing.py:7-144, vllm_rlt/kernels/metadata.py:7-24, the depth-table
  gather of vllm_rlt/worker/async_speculative.py:449-466), graph-capturable.

The directory is named ``vllm-rlt_amd``; it is imported as ``vllm_rlt_amd``
(see ``__graft_entry__.load_package``).
"""

from . import attention, kv_write, ops, routing, sampling  # noqa: F401
from .attention import (  # noqa: F401
    AttentionBackend,
    BackendCapabilities,
    MI355XPagedAttention,
    create_backend,
)
from .sampling import (  # noqa: F401
    AcceptResult,
    batched_probabilities,
    categorical,
    greedy_accept,
    greedy_accept_batched,
    merge_random_round,
    propose_drafts,
    RandomRoundMerge,
    rejection_round,
    rejection_rows,
    rejection_sample,
    speculative_accept,
    verify_accept,
    verify_distributions,
)
from .kv_write import (  # noqa: F401
    finalize_rows,
    masked_kv_store,
    store_fp8,
    store_kv,
    write_graph_kv,
)
