"""The attention oracle against closed forms (dense SDPA, single key, zero rows)."""

import pytest
import torch

from oracle import attention as oatt
from oracle import fp8 as ofp8
from tests.attn_cases import make_pool, random_tables


@pytest.mark.parametrize("head_dim,hq,hkv", [(7, 4, 2), (32, 6, 3), (128, 16, 4)])
def test_oracle_matches_dense_sdpa(head_dim, hq, hkv):
    g = torch.Generator().manual_seed(head_dim)
    bs = 5
    lengths = [1, 7, 31, 32, 70]
    _, _, k, v = make_pool(64, 3, bs, hkv, head_dim, torch.float32, g, layer=1)
    tables = random_tables(lengths, bs, 64, g)
    q = torch.randn(len(lengths), hq, head_dim, generator=g)
    got = oatt.paged_attention(q, k, v, tables, torch.tensor(lengths, dtype=torch.int32))
    for r, n in enumerate(lengths):
        pos = torch.arange(n)
        blocks = tables[r, pos // bs].long()
        kk, vv = k[blocks, pos % bs], v[blocks, pos % bs]
        torch.testing.assert_close(got[r], oatt.dense_attention(q[r], kk, vv), atol=1e-5, rtol=1e-5)


def test_oracle_single_key_and_empty_rows():
    g = torch.Generator().manual_seed(1)
    _, _, k, v = make_pool(8, 1, 16, 2, 32, torch.float32, g)
    tables = torch.tensor([[3], [5]], dtype=torch.int32)
    q = torch.randn(2, 4, 32, generator=g)
    out = oatt.paged_attention(q, k, v, tables, torch.tensor([1, 0], dtype=torch.int32))
    torch.testing.assert_close(out[0], v[3, 0].repeat_interleave(2, 0))  # softmax of one key = 1
    assert torch.count_nonzero(out[1]) == 0


def test_oracle_fp8_equals_dequantized():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(12, 16, 2, 32, generator=g)
    codes, scale = ofp8.quantize_fp8(x)
    err = (ofp8.dequantize_fp8(codes, scale, torch.float32) - x).abs()
    assert (err <= x.abs().amax(-1, keepdim=True) / 16 + 1e-30).all()
    tables = torch.tensor([[3, 1, 4]], dtype=torch.int32)
    q = torch.randn(1, 4, 32, generator=g)
    lengths = torch.tensor([40], dtype=torch.int32)
    got = oatt.paged_attention(q, codes, codes, tables, lengths, scale, scale)
    dense = ofp8.dequantize_fp8(codes, scale, torch.float32)
    torch.testing.assert_close(got, oatt.paged_attention(q, dense, dense, tables, lengths),
                               rtol=1e-5, atol=1e-6)
    fixed = torch.tensor(0.02)
    got = oatt.paged_attention(q, codes, codes, tables, lengths, fixed, fixed)
    dense = codes.float() * 0.02
    torch.testing.assert_close(got, oatt.paged_attention(q, dense, dense, tables, lengths),
                               rtol=1e-5, atol=1e-6)


def test_oracle_window_and_packed_layout():
    g = torch.Generator().manual_seed(3)
    _, _, k, v = make_pool(32, 1, 4, 2, 16, torch.float32, g)
    tables = random_tables([37, 9], 4, 32, g)
    lengths = torch.tensor([37, 9], dtype=torch.int32)
    cu = torch.tensor([0, 5, 8], dtype=torch.int32)
    seq, rl = oatt.packed_row_layout(lengths, cu)
    assert seq == [0] * 5 + [1] * 3 and rl == [33, 34, 35, 36, 37, 7, 8, 9]
    q = torch.randn(8, 4, 16, generator=g)
    packed = oatt.packed_window_attention(q, k, v, tables, lengths, cu, window=6)
    for r, (s, n) in enumerate(zip(seq, rl)):
        pos = torch.arange(max(0, n - 6), n)
        blocks = tables[s, pos // 4].long()
        torch.testing.assert_close(packed[r], oatt.dense_attention(q[r], k[blocks, pos % 4],
                                                                    v[blocks, pos % 4]),
                                   atol=1e-5, rtol=1e-5)
