"""The torch operator binding (``torch.ops.rlt_mi355x``): schemas, the absence of a
CPU kernel, and fake (shape) implementations, all without a GPU."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode


def test_operators_are_registered_with_reference_shaped_schemas(pkg):
    names = {op: str(getattr(torch.ops.rlt_mi355x, op).default._schema) for op in pkg.ops.OPS}
    assert "Tensor? cu_seqlens_q" in names["paged_attention"]
    assert names["spec_accept"].endswith("-> (Tensor, Tensor, Tensor, Tensor)")
    assert "!) key_cache" in names["store_kv"]
    assert "float? fixed_scale" in names["store_fp8"]
    assert "Tensor? row_lengths=None" in names["paged_attention"]
    assert "!) key_cache" in names["paged_attention_store"]
    assert names["merge_random_round"].endswith("-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)")


def test_per_step_operators_are_cpp(pkg):
    """The per-step entry points are the C++ operators of _C.so (TORCH_LIBRARY in
    csrc/torch_bindings.cpp), not Python custom ops."""
    import os

    from vllm_rlt_amd import _lib

    assert os.path.exists(_lib.OPS_PATH)
    for op in ("paged_attention", "paged_attention_store", "store_kv", "spec_probs", "categorical", "spec_accept",
               "greedy_accept", "verify_distributions", "verify_accept"):
        kernels = torch._C._dispatch_dump(f"rlt_mi355x::{op}")
        assert "CUDA: registered at" in kernels and "torch_bindings.cpp" in kernels, op


def test_cpu_tensors_find_no_kernel(pkg):
    with pytest.raises(NotImplementedError, match="CPU"):
        torch.ops.rlt_mi355x.spec_probs(torch.zeros(2, 5), torch.ones(2),
                                        torch.zeros(2, dtype=torch.long), torch.ones(2), 0, False)
    with pytest.raises(NotImplementedError, match="CPU"):
        torch.ops.rlt_mi355x.categorical(torch.ones(2, 5), torch.zeros(2))


def test_fake_implementations_give_output_shapes(pkg):
    with FakeTensorMode():
        q = torch.empty(10, 16, 128, dtype=torch.bfloat16)
        kc = torch.empty(64, 16, 4, 128, dtype=torch.bfloat16)
        out = torch.ops.rlt_mi355x.paged_attention(
            q, kc, kc, torch.empty(2, 8, dtype=torch.int32), torch.empty(2, dtype=torch.int32),
            None, None, torch.empty(3, dtype=torch.int32), 5, 0)
        assert out.shape == q.shape and out.dtype == q.dtype
        p = torch.ops.rlt_mi355x.spec_probs(torch.empty(6, 1000, dtype=torch.bfloat16),
                                            torch.empty(6), torch.empty(6, dtype=torch.int64),
                                            torch.empty(6), 0, True)
        assert p.shape == (6, 1000) and p.dtype == torch.float32
        toks, acc, fin, err = torch.ops.rlt_mi355x.spec_accept(
            torch.empty(3, 4, dtype=torch.int64), torch.empty(3, dtype=torch.int64),
            torch.empty(3, 4, 50), torch.empty(3, 5, 50), torch.empty(3, 4), torch.empty(3))
        assert toks.shape == (3, 5) and acc.shape == fin.shape == err.shape == (3,)
        assert err.dtype == torch.bool
        prop, q_o = torch.ops.rlt_mi355x.propose_drafts(
            torch.empty(7, 300), torch.empty(2, dtype=torch.int64), torch.empty(2),
            torch.empty(2, dtype=torch.int64), torch.empty(2), torch.empty(2), 0, False)
        assert prop.shape == (7,) and q_o.shape == (2, 300)
        out = torch.ops.rlt_mi355x.verify_accept(
            torch.empty(3, 5, 80), torch.empty(15), torch.empty(15, dtype=torch.int64),
            torch.empty(15), torch.empty(3, 4, dtype=torch.int64),
            torch.empty(3, dtype=torch.int64), torch.empty(3, 4, 80), torch.empty(3, 4),
            torch.empty(3), 0, True)
        assert [tuple(x.shape) for x in out] == [(15,), (3, 5, 80), (3, 5), (3,), (3,), (3,)]
