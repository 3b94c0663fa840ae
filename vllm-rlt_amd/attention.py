"""MI355X paged-attention backend behind the reference attention-backend interface.

Mirrors vllm_rlt/attention/backend.py (``BackendCapabilities`` :19-36,
``AttentionBackend`` :40-83, ``create_backend`` :177-276) and the kernel-object
protocol of vllm_rlt/kernels/paged_attention.py (``__call__`` / ``windowed`` /
``prefill``), so the KV cache manager's call sites
(vllm_rlt/core/kv_cache_manager.py:993-1018) and the graph-time call site
(vllm_rlt/worker/cuda_graph.py:161-167) drive it unchanged.

Every call goes through the C++ operator ``torch.ops.rlt_mi355x.paged_attention``
(csrc/torch_bindings.cpp), which launches the gfx950 kernels of librlt_mi355x.so
on the current HIP stream: no host synchronization, no fallback, static grids (capturable in HIP
graphs).  The per-row, windowed and packed forms share one kernel whose per-row
arithmetic is independent of batch composition, which is why this backend can
declare ``packed_matches_decode``.
"""

import logging
from dataclasses import dataclass, replace

import torch

from . import _lib


@dataclass(frozen=True)
class BackendCapabilities:
    """Execution features; field meanings follow vllm_rlt/attention/backend.py:19-36."""

    packed_prefill: bool = False
    cuda_graphs: bool = False
    async_scheduling: bool = False
    packed_matches_decode: bool = False
    fp8_kv: bool = False
    fp8_kv_static: bool = False
    device_context_lengths: bool = False
    sliding_window: bool = False
    packed_sliding_window: bool = False


@dataclass
class AttentionBackend:
    """Kernel adapter with declared features; reference: backend.py:40-83."""

    kernel: object
    capabilities: BackendCapabilities
    info: dict

    def __call__(self, *args, **kwargs):
        return self.kernel(*args, **kwargs)

    def attend_metadata(self, q, keys, values, batch, **kwargs):
        method = getattr(self.kernel, "attend_metadata", None)
        if method is not None:
            return method(q, keys, values, batch, **kwargs)
        if getattr(batch, "cu_seqlens_q", None) is not None:
            return self.prefill(q, keys, values, batch.block_tables, batch.context_lengths,
                                batch.cu_seqlens_q, batch.max_seqlen_q, **kwargs)
        return self(q, keys, values, batch.block_tables, batch.context_lengths, **kwargs)

    def prefill(self, *args, **kwargs):
        return self.kernel.prefill(*args, **kwargs)

    def prefill_store(self, *args, **kwargs):
        return self.kernel.prefill_store(*args, **kwargs)

    def windowed(self, *args, **kwargs):
        method = getattr(self.kernel, "windowed", None)
        if method is None:
            selected = self.info.get("selected_backend", "this attention backend")
            raise NotImplementedError(f"{selected} does not implement sliding-window masking")
        return method(*args, **kwargs)

    @property
    def generation(self):
        return getattr(self.kernel, "generation", None)


MI355X_CAPABILITIES = BackendCapabilities(
    packed_prefill=True,
    cuda_graphs=True,
    async_scheduling=True,
    packed_matches_decode=True,
    fp8_kv=True,
    fp8_kv_static=True,
    device_context_lengths=True,
    sliding_window=True,
    packed_sliding_window=True,
)


class MI355XPagedAttention:
    """Split-KV paged GQA attention on gfx950 (per-row, windowed and packed forms).

    ``compensate``: as the reference's ``TritonPagedAttention(compensate=True)``
    (vllm_rlt/kernels/triton_attention.py:368-371), the 16-bit cast of the softmax
    weights for the P V product is followed by a second MFMA with the bits it dropped,
    so P V keeps ~16 bits of each weight instead of 8 (bf16).  Applies to bf16 / fp16
    q on pools whose block size is a multiple of 16; packed calls then stay on the
    verify kernels at every window length (rows equal per-row rows bit for bit).
    """

    generation = None

    def __init__(self, compensate=False):
        self.compensate = bool(compensate)

    def _run(self, q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q,
             max_seqlen_q, key_scale, value_scale, window, row_lengths=None):
        if type(window) is not int or window < 0:
            raise ValueError("window must be a nonnegative integer")
        _lib.require_gpu(q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q,
                         key_scale, value_scale, row_lengths)
        # argument checks, workspace and launch: torch.ops.rlt_mi355x.paged_attention
        # (csrc/torch_bindings.cpp), ValueError on a bad argument
        return _lib.ops().paged_attention(q, key_cache, value_cache, block_tables,
                                          context_lengths, key_scale, value_scale, cu_seqlens_q,
                                          int(max_seqlen_q) if cu_seqlens_q is not None else 1,
                                          window, row_lengths, self.compensate)

    def __call__(self, q, key_cache, value_cache, block_tables, context_lengths,
                 key_scale=None, value_scale=None):
        """Per-row decode / verify; reference: kernels/paged_attention.py:13-47, :210-220."""
        return self._run(q, key_cache, value_cache, block_tables, context_lengths, None, 1,
                         key_scale, value_scale, 0)

    def windowed(self, q, key_cache, value_cache, block_tables, context_lengths, window,
                 key_scale=None, value_scale=None):
        """Last-``window``-keys masking; reference: kernels/paged_attention.py:50-90."""
        if isinstance(window, bool) or not isinstance(window, int) or window <= 0:
            raise ValueError("window must be a positive integer")
        return self._run(q, key_cache, value_cache, block_tables, context_lengths, None, 1,
                         key_scale, value_scale, window)

    def prefill(self, q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q,
                max_seqlen_q, key_scale=None, value_scale=None, *, window=0, row_lengths=None):
        """Packed causal window, bottom-right aligned; reference: triton_attention.py:386-404.

        ``row_lengths`` (int32 ``[q rows]``, optional, not in the reference signature): row i
        of a sequence sees ``row_lengths[cu_seqlens_q[s] + i]`` keys instead of the causal
        window's ``context_lengths[s] - q_len + i + 1``, in any order.  Rows that read one block table at non-consecutive positions
        (pipelined verify rows at the same loop-depth plane) then share each KV byte, and
        every row equals the per-row ``__call__`` bit for bit.
        """
        return self._run(q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q,
                         max_seqlen_q, key_scale, value_scale, window, row_lengths)

    def prefill_store(self, q, k_new, v_new, key_cache, value_cache, block_tables,
                      context_lengths, cu_seqlens_q, max_seqlen_q, key_scale=None,
                      value_scale=None, *, row_lengths=None):
        """Store the window rows' own keys / values, then ``prefill`` (no sliding window).

        ``k_new`` / ``v_new`` ``[q rows, kv_heads, head_dim]``: row r is written into the
        pool at packed q row r's position (``context_lengths[s] - q_len + i`` for window row
        i of sequence s, or ``row_lengths[r] - 1`` with explicit row lengths) through
        ``block_tables`` -- the KV write that precedes attention in every layer (reference:
        vllm_rlt/kernels/graph_kv.py:52-67; for FP8 pools the quantize-store
        vllm_rlt/kernels/triton_attention.py:506-623) -- and the attention then reads it.
        FP8 pools take bf16 / fp16 rows and quantize them as ``store_fp8`` does: with the
        0-d per-tensor ``key_scale`` / ``value_scale`` (only read), or with per-vector
        scales written into the ``[block, token, kv_head]`` scale views.  Verify windows on
        the MFMA kernels run as one launch pair (the attention waves that read a window
        position store it first); other 16-bit shapes store with ``store_kv`` and attend
        separately.  Returns the attention output.
        """
        _lib.require_gpu(q, k_new, v_new, key_cache, value_cache, block_tables, context_lengths,
                         cu_seqlens_q, key_scale, value_scale, row_lengths)
        # argument checks, the one-launch form or the separate store + attention:
        # torch.ops.rlt_mi355x.paged_attention_store (csrc/torch_bindings.cpp)
        return _lib.ops().paged_attention_store(q, k_new, v_new, key_cache, value_cache,
                                                block_tables, context_lengths, cu_seqlens_q,
                                                int(max_seqlen_q), key_scale, value_scale,
                                                row_lengths, self.compensate)

    def uses_mfma(self, q_dtype, kv_dtype, head_dim):
        lib = _lib.library()
        return bool(lib.rlt_paged_attention_uses_mfma(_lib.dtype_code(q_dtype),
                                                      _lib.dtype_code(kv_dtype), head_dim))

    def uses_prefill_tiling(self, q_dtype, kv_dtype, head_dim, max_seqlen_q):
        """True when ``prefill`` calls with this longest window take the long-prompt
        tiling (equal to the per-row form within tolerance, not bit for bit)."""
        lib = _lib.library()
        return bool(lib.rlt_paged_attention_uses_prefill(
            _lib.dtype_code(q_dtype), _lib.dtype_code(kv_dtype), head_dim, max_seqlen_q))


_BACKEND_NAMES = ("auto", "mi355x")


def create_backend(backend, device, dtype, head_dim, block_size, *,
                   required_capabilities=BackendCapabilities(), prefer_packed_prefill=False,
                   packed_window_shape=None, allow_fp8_calibration=False):
    """Select the MI355X backend; explicit failures, no silent fallback.

    reference: vllm_rlt/attention/backend.py:177-276.  There is exactly one
    implementation, so ``auto`` and ``mi355x`` are the same choice; any other
    name, a non-ROCm device, head_dim > 256 or a missing capability raises.
    """
    if backend not in _BACKEND_NAMES:
        raise ValueError("unknown attention backend")
    device = torch.device(device)
    if device.type != "cuda" or torch.version.hip is None:
        raise ValueError("the MI355X attention backend requires a ROCm device")
    if head_dim > 256:
        raise ValueError("the MI355X attention backend supports head_dim <= 256")
    if dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError(f"unsupported attention dtype {dtype}")
    _lib.library()  # fail at selection time, before the KV pool is allocated
    capabilities = MI355X_CAPABILITIES
    names = ("packed_prefill", "cuda_graphs", "async_scheduling", "device_context_lengths",
             "fp8_kv", "fp8_kv_static", "sliding_window", "packed_sliding_window")
    missing = [n for n in names
               if getattr(required_capabilities, n) and not getattr(capabilities, n)]
    if missing:
        raise ValueError(f"mi355x lacks required capabilities: {', '.join(missing)}")
    # a packed window shape opts into the compensated P V product for bf16, as the
    # reference's packed-window tile selection does (vllm_rlt/attention/backend.py:146-161,
    # kernels/triton_attention.py:626-628); the blocks must hold whole 16-position tiles
    compensate = (packed_window_shape is not None and dtype == torch.bfloat16 and
                  block_size % 16 == 0)
    kernel = MI355XPagedAttention(compensate=compensate)
    info = {
        "backend": "mi355x",
        "requested_backend": backend,
        "selected_backend": "mi355x",
        "selection_reason": "single gfx950 implementation",
        "math": "mfma" if kernel.uses_mfma(dtype, dtype, head_dim) else "vector",
        "compensated_p": compensate,
    }
    logging.getLogger(__name__).info("Attention selection: %s", info)
    return AttentionBackend(kernel, replace(capabilities), info)
