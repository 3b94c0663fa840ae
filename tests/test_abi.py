"""The C ABI: the library loads, exports every declared entry point, and its
host-side argument checks answer without a GPU."""

import ctypes
import os
import re

import pytest

from tests.conftest import ROOT


def _declared():
    text = open(os.path.join(ROOT, "include", "rlt_mi355x.h")).read()
    return sorted(set(re.findall(r"^(?:size_t|int)\s+(rlt_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol(pkg):
    from vllm_rlt_amd import _lib

    lib = _lib.library()
    declared = _declared()
    assert len(declared) >= 9
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.EXPORTED)


def test_workspace_queries_are_host_only(pkg):
    from vllm_rlt_amd import _lib

    lib = _lib.library()
    assert lib.rlt_speculative_accept_workspace_size(32, 4, 49152) > 0
    assert lib.rlt_categorical_workspace_size(8, 65536) > 0
    # the row-split distributions: workspace for V up to 16 slices of 16384 columns
    assert lib.rlt_probabilities_workspace_size(160, 0, 49152) > 0
    assert lib.rlt_probabilities_workspace_size(160, 160, 49152) > \
        lib.rlt_probabilities_workspace_size(160, 0, 49152)
    assert lib.rlt_probabilities_workspace_size(8, 0, 262144) > 0
    assert lib.rlt_probabilities_workspace_size(8, 0, 262145) == 0
    assert lib.rlt_verify_accept_workspace_size(32, 4, 49152) > \
        lib.rlt_speculative_accept_workspace_size(32, 4, 49152)
    assert lib.rlt_propose_drafts_workspace_size(256, 32, 49152) > \
        lib.rlt_categorical_workspace_size(32, 49152)
    # 160 rows x 16 heads x (512 blocks x 16 / 512 chunks) x (2 + 128) floats
    n = lib.rlt_paged_attention_workspace_size(160, 16, 128, 512, 16)
    assert n >= 160 * 16 * 16 * 130 * 4
    assert lib.rlt_paged_attention_uses_mfma(2, 2, 128) == 1
    assert lib.rlt_paged_attention_uses_mfma(2, 3, 96) == 1
    assert lib.rlt_paged_attention_uses_mfma(0, 0, 128) == 0
    assert lib.rlt_paged_attention_uses_mfma(2, 2, 7) == 0
    assert lib.rlt_paged_attention_uses_prefill(2, 2, 128, 64) == 1
    assert lib.rlt_paged_attention_uses_prefill(2, 2, 128, 33) == 0  # verify windows
    assert lib.rlt_paged_attention_uses_prefill(2, 3, 128, 512) == 1  # fp8 pools
    assert lib.rlt_paged_attention_uses_prefill(2, 2, 96, 512) == 1  # padded LDS rows
    assert lib.rlt_paged_attention_uses_prefill(2, 2, 256, 512) == 0


def test_argument_errors_return_status_without_launching(pkg):
    from vllm_rlt_amd import _lib

    lib = _lib.library()
    null = ctypes.c_void_p(0)
    # q heads not a multiple of kv heads -> RLT_ERR_ARGUMENT (1)
    st = lib.rlt_paged_attention(null, 0, 0, null, null, 0, 0, 0, 0, 0, 0, 1, null, 0, 1, null,
                                 null, 1, 1, 1, null, null, 0, 0, 0, 0, 6, 4, 128, 16, 2, 2, 0,
                                 null, 0, 0, null, 0, null)
    assert st == 1
    # missing workspace -> RLT_ERR_WORKSPACE (3)
    st = lib.rlt_speculative_accept(null, null, null, null, null, null, 4, 4, 1000, null, null, null,
                                    null, null, 0, null)
    assert st == 3
    # vocabulary too large -> RLT_ERR_UNSUPPORTED (2)
    st = lib.rlt_speculative_accept(null, null, null, null, null, null, 4, 4, 1 << 25, null, null,
                                    null, null, null, 0, null)
    assert st == 2


def test_host_api_validates_before_touching_a_device(pkg):
    import torch

    with pytest.raises(ValueError):
        pkg.create_backend("triton", torch.device("cpu"), torch.bfloat16, 128, 16)
    with pytest.raises(ValueError):
        pkg.create_backend("auto", torch.device("cpu"), torch.bfloat16, 128, 16)
    with pytest.raises(ValueError):
        pkg.speculative_accept(torch.zeros(2, 3, dtype=torch.long), torch.zeros(3, dtype=torch.long),
                               torch.zeros(2, 3, 4), torch.zeros(2, 4, 4), torch.zeros(2, 3),
                               torch.zeros(2))
    with pytest.raises(ValueError):
        pkg.categorical(torch.zeros(2, 4), torch.zeros(2))  # CPU tensors are refused
    with pytest.raises(ValueError, match="window"):
        pkg.MI355XPagedAttention().windowed(None, None, None, None, None, 0)


def test_probability_and_greedy_entry_points_check_arguments(pkg):
    from vllm_rlt_amd import _lib

    lib = _lib.library()
    null, fake = ctypes.c_void_p(0), ctypes.c_void_p(16)
    # negative rows / row stride below V -> RLT_ERR_ARGUMENT (1)
    assert lib.rlt_batched_probabilities(null, 0, 10, -1, 10, null, null, null, 0, 0, null, 10,
                                         null, 0, null) == 1
    assert lib.rlt_batched_probabilities(fake, 0, 5, 2, 10, fake, fake, fake, 0, 0, fake, 10,
                                         null, 0, null) == 1
    # zero rows: nothing to launch
    assert lib.rlt_batched_probabilities(null, 0, 10, 0, 10, null, null, null, 0, 0, null, 10,
                                         null, 0, null) == 0
    # missing pointers -> 1; V above 262144 -> RLT_ERR_UNSUPPORTED (2); fp8 logits -> 2
    assert lib.rlt_batched_probabilities(null, 0, 10, 2, 10, fake, fake, fake, 0, 0, fake, 10,
                                         null, 0, null) == 1
    big = 262144 + 1
    assert lib.rlt_batched_probabilities(fake, 0, big, 2, big, fake, fake, fake, 0, 0, fake, big,
                                         null, 0, null) == 2
    assert lib.rlt_batched_probabilities(fake, 3, 10, 2, 10, fake, fake, fake, 0, 0, fake, 10,
                                         null, 0, null) == 2
    # a workspace smaller than the row-split form's query -> RLT_ERR_WORKSPACE (3)
    assert lib.rlt_batched_probabilities(fake, 0, 10, 2, 10, fake, fake, fake, 0, 0, fake, 10,
                                         fake, 1, null) == 3
    assert lib.rlt_greedy_accept(null, null, null, 0, 10, -1, 4, 10, null, null, null, null) == 1
    assert lib.rlt_greedy_accept(fake, fake, fake, 0, 5, 2, 4, 10, fake, fake, fake, null) == 1
    assert lib.rlt_greedy_accept(fake, fake, fake, 3, 10, 2, 4, 10, fake, fake, fake, null) == 2
    assert lib.rlt_greedy_accept(null, null, null, 0, 10, 0, 4, 10, null, null, null, null) == 0


def test_probability_host_api_refuses_cpu_tensors(pkg):
    import torch

    x = torch.zeros(2, 8)
    with pytest.raises(ValueError):
        pkg.batched_probabilities(x, torch.ones(2), torch.zeros(2, dtype=torch.long),
                                  torch.ones(2), max_top_k=0, apply_top_p=False)
    with pytest.raises(ValueError):
        pkg.greedy_accept_batched(torch.zeros(2, 4, dtype=torch.long),
                                  torch.zeros(2, dtype=torch.long), torch.zeros(2, 5, 8))


def test_kv_write_entry_points_check_arguments(pkg):
    from vllm_rlt_amd import _lib

    lib = _lib.library()
    null, fake = None, 0x1000
    # rlt_kv_store: zero rows is a no-op; bad heads / dtype / block size are refused
    args = [fake, fake, 8, 4, 8, 4, fake, fake, 64, 8, 4, 10, 8, fake, fake, null, null]
    assert lib.rlt_kv_store(*args, 0, 2, 4, 2, null) == 0
    assert lib.rlt_kv_store(*args, 3, 0, 4, 2, null) == 1
    assert lib.rlt_kv_store(*args, 3, 2, 4, 9, null) == 1
    assert lib.rlt_kv_store(*args[:6], null, fake, *args[8:], 3, 2, 4, 2, null) == 1
    # rlt_kv_store_fp8: head_dim above one wave's 256 elements is unsupported
    fp8 = [fake, fake, 2, 8, 4, 8, 4, fake, fake, 64, 8, 4, fake, fake, 16, 2, 1, 10, 8,
           fake, fake, null, null]
    assert lib.rlt_kv_store_fp8(*fp8, 0, 2, 4, 0, 0.0, null) == 0
    assert lib.rlt_kv_store_fp8(*fp8, 3, 2, 512, 0, 0.0, null) == 2
    assert lib.rlt_kv_store_fp8(*fp8[:12], null, *fp8[13:], 3, 2, 4, 0, 0.0, null) == 1
    # rlt_kv_finalize: one plane has nothing deeper to copy into
    fin = [fake, 4, fake, 2, 8]
    assert lib.rlt_kv_finalize(*fin, 1, 16, 2, 10, fake, fake, 64, 32, 4, 4, 1, null) == 0
    assert lib.rlt_kv_finalize(*fin, 4, 0, 2, 10, fake, fake, 64, 32, 4, 4, 1, null) == 1
    assert lib.rlt_kv_finalize(*fin[:2], null, *fin[3:], 4, 16, 2, 10, fake, fake, 64, 32, 4,
                               4, 1, null) == 1


def test_kv_write_host_api_refuses_cpu_tensors(pkg):
    import torch

    from vllm_rlt_amd import kv_write

    pool = torch.zeros(4, 8, 2, 16, dtype=torch.bfloat16)
    rows = torch.zeros(3, 2, 16, dtype=torch.bfloat16)
    idx = torch.zeros(3, dtype=torch.long)
    with pytest.raises(ValueError, match="ROCm"):
        kv_write.store_kv(pool, pool.clone(), rows, rows, idx, idx)
    with pytest.raises(ValueError, match="pool's dtype"):
        kv_write.store_kv(pool, pool.clone(), rows.float(), rows.float(), idx, idx)
    codes = torch.zeros(4, 8, 2, 16, dtype=torch.float8_e4m3fn)
    scale = torch.ones(4, 8, 2)
    with pytest.raises(ValueError, match="448"):
        kv_write.store_fp8(rows, rows, codes, codes, scale, scale, idx, idx, 240.0)
    with pytest.raises(ValueError, match="ROCm"):
        kv_write.store_fp8(rows, rows, codes, codes, scale, scale, idx, idx, 448.0)
    with pytest.raises(ValueError, match="descriptor"):
        kv_write.finalize_rows(torch.zeros(2, 2), torch.zeros(1, 2, 3), pool, pool, 8)


def test_routing_entry_points_check_arguments(pkg):
    from vllm_rlt_amd import _lib

    lib = _lib.library()
    null, fake = None, 0x1000
    assert lib.rlt_route_slots(null, fake, 0, 0, null) == 0  # empty: no launch
    assert lib.rlt_route_slots(fake, fake, 5, 4, null) == 1  # count > size
    assert lib.rlt_route_metadata(fake, fake, 8, 4, 16, 2, *[fake] * 6, 4, 5, 1, 1, null) == 1
    assert lib.rlt_route_metadata(fake, fake, 8, 4, 16, 2, *[fake] * 6, 4, 4, 0, 0, null) == 0
    assert lib.rlt_route_metadata(null, null, 8, 4, 16, 2, *[fake] * 6, 4, 4, 0, 3, null) != 1
    assert lib.rlt_route_gather(fake, 4, 8, fake, fake, 4, 1, 2, 8, 2, null) == 1  # stride < row
    assert lib.rlt_route_scatter(fake, 8, fake, fake, 4, 8, 0, 8, 2, null) == 0
    assert lib.rlt_route_gather_segments(fake, 2, 4, 8, fake, 3, 70000, fake, 9, 8, 8, 2,
                                         null) == 2  # grid y beyond 65535
    assert lib.rlt_route_scatter_segments(fake, 4, 8, null, 3, 2, fake, 2, 4, 8, 8, 2, null) == 1
    assert lib.rlt_expand_kv_addresses(fake, fake, fake, 4, 0, 16, fake, fake, 3, null) == 1
    assert lib.rlt_depth_tables(fake, 8, 4, 2, 4, fake, fake, null, 16, fake, 2, fake, fake,
                                fake, 3, null) == 1  # out_stride < width


def test_propose_drafts_checks_arguments(pkg):
    from vllm_rlt_amd import _lib

    lib = _lib.library()
    null, fake = None, 0x1000
    base = [fake, 0, 100, 4, 100]
    # nothing to do
    assert lib.rlt_propose_drafts(fake, 0, 100, 0, 100, null, 0, null, null, null, 0, 0, null,
                                  null, 100, fake, null, 0, null) == 0
    # random rows without their per-row arguments
    assert lib.rlt_propose_drafts(*base, fake, 2, null, null, null, 0, 0, null, null, 100, fake,
                                  null, 0, null) == 1
    # workspace too small for the draws
    assert lib.rlt_propose_drafts(*base, fake, 2, fake, fake, fake, 0, 0, fake, fake, 100, fake,
                                  fake, 1, null) == 3
    # q rows narrower than the vocabulary
    assert lib.rlt_propose_drafts(*base, fake, 2, fake, fake, fake, 0, 0, fake, fake, 50, fake,
                                  fake, 1 << 20, null) == 1


def test_verify_accept_checks_arguments(pkg):
    from vllm_rlt_amd import _lib

    lib = _lib.library()
    null, fake = None, 0x1000
    io = [fake] * 6  # targets, p_out, tokens, accepted, final_token, error
    # nothing to do
    assert lib.rlt_verify_accept(fake, 0, 100, fake, fake, fake, 0, 0, null, fake, null, null,
                                 fake, 0, 4, 100, *io, null, 0, null) == 0
    # row stride narrower than the vocabulary
    assert lib.rlt_verify_accept(fake, 0, 50, fake, fake, fake, 0, 0, fake, fake, fake, fake,
                                 fake, 2, 4, 100, *io, fake, 1 << 20, null) == 1
    # drafts without draft tokens / q / uniforms
    assert lib.rlt_verify_accept(fake, 0, 100, fake, fake, fake, 0, 0, null, fake, null, null,
                                 fake, 2, 4, 100, *io, fake, 1 << 20, null) == 1
    # more than 32 drafts per request
    assert lib.rlt_verify_accept(fake, 0, 100, fake, fake, fake, 0, 0, fake, fake, fake, fake,
                                 fake, 2, 33, 100, *io, fake, 1 << 30, null) == 2
    # workspace too small
    assert lib.rlt_verify_accept(fake, 0, 100, fake, fake, fake, 0, 0, fake, fake, fake, fake,
                                 fake, 2, 4, 100, *io, fake, 1, null) == 3


def test_attention_with_window_store_checks_arguments(pkg):
    """rlt_paged_attention_store serves packed bf16 / fp16 windows only: other forms
    return RLT_ERR_UNSUPPORTED (2) and a missing or misaligned window buffer
    RLT_ERR_ARGUMENT (1), before anything is launched."""
    from vllm_rlt_amd import _lib

    lib = _lib.library()
    null, fake = None, 0x1000
    hq, hkv, d, bs = 16, 4, 128, 16

    def call(cu=fake, max_q=5, dtype=2, new_k=fake, new_v=fake, row_stride=hkv * d, seqs=2):
        # q, pools [block, token, kv_head, dim] with 64 blocks, 2 sequences x 5 rows
        return lib.rlt_paged_attention_store(
            fake, hq * d, d, fake, fake, bs * hkv * d, hkv * d, d, bs * hkv * d, hkv * d, d, 64,
            fake, 8, 8, fake, cu, seqs, max_q, 10, hq, hkv, d, bs, dtype, new_k, new_v, row_stride,
            d, fake, hq * d, d, fake, 1 << 24, null)

    assert call(cu=null, seqs=10) == 2  # per-row form: no window to store
    assert call(dtype=0) == 2          # float32 q and pool
    assert call(new_k=null) == 1       # no rows to store
    assert call(max_q=64, new_k=null) == 1  # prefill-length windows (store kernel + tiling) too
    assert call(new_v=fake + 2) == 1   # misaligned rows
    assert call(row_stride=hkv * d + 1) == 1
