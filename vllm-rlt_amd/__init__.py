"""vllm_rlt_amd -- MI355X-native speculative-verification hot path of vllm-rlt.

Drop-in host layer over ``librlt_mi355x.so`` (hand-written gfx950 HIP kernels):

* ``attention``: ``BackendCapabilities`` / ``AttentionBackend`` / ``create_backend``
  and the ``MI355XPagedAttention`` kernel object with the reference's per-row
  ``__call__``, ``windowed`` and packed ``prefill`` signatures
  (vllm_rlt/attention/backend.py, vllm_rlt/kernels/paged_attention.py).
* ``sampling``: ``batched_probabilities``, ``categorical``, ``speculative_accept`` /
  ``AcceptResult``, ``greedy_accept`` and the device greedy round
  ``greedy_accept_batched`` (vllm_rlt/worker/speculative_sampling.py,
  vllm_rlt/worker/speculative.py:41-53, vllm_rlt/worker/async_speculative.py:706-720).

The directory is named ``vllm-rlt_amd``; it is imported as ``vllm_rlt_amd``
(see ``__graft_entry__.load_package``).
"""

from . import attention, sampling  # noqa: F401
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
    speculative_accept,
)
