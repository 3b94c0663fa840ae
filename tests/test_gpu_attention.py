"""gfx950 paged attention against the CPU oracle (parity), bitwise invariants,
and the reference's edge cases.  Tolerances: bf16 2e-2 abs, fp16 2e-3, fp32
1e-5 (rel and abs)."""

import math
import sys

import pytest
import torch

from oracle import attention as oatt
from oracle import fp8 as ofp8
from tests.attn_cases import make_pool, random_tables

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 2e-2}


def _say(*args):
    print("[case]", *args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def kernel(pkg, dev):
    return pkg.MI355XPagedAttention()


def _close(got, want, dtype):
    tol = TOL[dtype]
    torch.testing.assert_close(got.float().cpu(), want.float(), atol=tol, rtol=tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [7, 32, 64, 96, 128])
def test_mixed_depth_rows_match_oracle(kernel, dev, dtype, head_dim):
    # reference shape: tests/test_attention.py:21-48 (mixed requests and depths on a
    # fragmented pool, 6 q heads over 2 kv heads, block size 3)
    _say("mixed", dtype, head_dim)
    g = torch.Generator().manual_seed(48 + head_dim)
    bs, hkv, hq = 3, 2, 6
    kpool, vpool, k, v = make_pool(80, 2, bs, hkv, head_dim, dtype, g, layer=1)
    lengths = [7, 5, 3, 6, 1, 33, 0, 64]
    tables = random_tables(lengths, bs, 80, g)
    q = torch.randn(len(lengths), hq, head_dim, generator=g).to(dtype)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    got = kernel(q.to(dev), kpool.to(dev)[:, 1], vpool.to(dev)[:, 1], tables.to(dev), ctx.to(dev))
    want = oatt.paged_attention(q, k, v, tables, ctx)
    _close(got, want, dtype)
    assert torch.count_nonzero(got[6]) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_split_kv_lengths_and_batch_invariance(kernel, dev, dtype):
    # reference: tests/test_attention.py:154-184
    _say("split", dtype)
    g = torch.Generator().manual_seed(1)
    bs, hq, hkv, d = 16, 8, 4, 128
    lengths = [0, 1, 31, 32, 33, 511, 512, 513, 4097, 10000]
    pages = sum(-(-n // bs) for n in lengths)
    _, _, k, v = make_pool(pages, 1, bs, hkv, d, dtype, g)
    tables = random_tables(lengths, bs, pages, g)
    q = torch.randn(len(lengths), hq, d, generator=g).to(dtype)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    kd, vd, td, cd, qd = k.to(dev), v.to(dev), tables.to(dev), ctx.to(dev), q.to(dev)
    got = kernel(qd, kd, vd, td, cd)
    _close(got, oatt.paged_attention(q, k, v, tables, ctx), dtype)
    assert torch.count_nonzero(got[0]) == 0
    for row in (1, 5, 8, 9):
        alone = kernel(qd[row:row + 1], kd, vd, td[row:row + 1], cd[row:row + 1])
        assert torch.equal(alone[0], got[row])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("head_dim,heads,kv_heads", [(64, 4, 2), (96, 8, 8), (128, 16, 4),
                                                     (128, 16, 16)])
def test_packed_window_matches_oracle_and_per_row_bitwise(kernel, dev, dtype, head_dim, heads,
                                                          kv_heads):
    # reference: tests/test_attention.py:110-151 (prefixes 32, 0, 0, 60, 9; pages out of order)
    _say("packed", dtype, head_dim, heads, kv_heads)
    g = torch.Generator().manual_seed(0)
    bs = 16
    seqs = [(37, 5), (100, 100), (3, 3), (130, 70), (129, 120), (700, 5), (5, 5)]
    pages = sum(-(-n // bs) for n, _ in seqs) + 3
    _, _, k, v = make_pool(pages, 1, bs, kv_heads, head_dim, dtype, g)
    tables = random_tables([n for n, _ in seqs], bs, pages, g)
    total = sum(c for _, c in seqs)
    q = torch.randn(total, heads, head_dim, generator=g).to(dtype)
    lengths = torch.tensor([n for n, _ in seqs], dtype=torch.int32)
    cu = torch.tensor([0] + list(torch.tensor([c for _, c in seqs]).cumsum(0)), dtype=torch.int32)
    kd, vd = k.to(dev), v.to(dev)
    packed = kernel.prefill(q.to(dev), kd, vd, tables.to(dev), lengths.to(dev), cu.to(dev),
                            max(c for _, c in seqs))
    want = oatt.packed_window_attention(q, k, v, tables, lengths, cu)
    _close(packed, want, dtype)
    seq_of_row, row_len = oatt.packed_row_layout(lengths, cu)
    per_row = kernel(q.to(dev), kd, vd, tables[torch.tensor(seq_of_row)].to(dev),
                     torch.tensor(row_len, dtype=torch.int32).to(dev))
    if kernel.uses_prefill_tiling(dtype, dtype, head_dim, max(c for _, c in seqs)):
        # windows of 64+ rows take the prefill tiling: equal within tolerance
        _close(packed, per_row.cpu().float(), dtype)
    else:
        assert torch.equal(per_row, packed), "packed window differs from per-row decode"
    # verify-length windows (at most 33 rows) equal per-row decode bit for bit
    short = torch.tensor([0, 5, 38, 41, 58, 91, 96, 101], dtype=torch.int32)
    assert not kernel.uses_prefill_tiling(dtype, dtype, head_dim, 33)
    qs = q[: int(short[-1])]
    packed_s = kernel.prefill(qs.to(dev), kd, vd, tables.to(dev), lengths.to(dev), short.to(dev),
                              33)
    seq_of_row, row_len = oatt.packed_row_layout(lengths, short)
    per_row_s = kernel(qs.to(dev), kd, vd, tables[torch.tensor(seq_of_row)].to(dev),
                       torch.tensor(row_len, dtype=torch.int32).to(dev))
    assert torch.equal(per_row_s, packed_s), "packed verify window differs from per-row decode"


@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("fixed", [False, True])
def test_fp8_pool_matches_oracle(kernel, dev, q_dtype, fixed):
    # reference: tests/test_fp8_kv_cache.py:69-84, :235-262
    _say("fp8", q_dtype, fixed)
    g = torch.Generator().manual_seed(5)
    bs, hkv, hq, d, layers = 16, 2, 8, 128, 2
    lengths = [1, 17, 300, 1025]
    pages = sum(-(-n // bs) for n in lengths)
    x = torch.randn(pages, layers, bs, hkv, d, generator=g) * 3
    y = torch.randn(pages, layers, bs, hkv, d, generator=g)
    kc, ks = ofp8.quantize_fp8(x, 0.05 if fixed else None)
    vc, vs = ofp8.quantize_fp8(y, 0.02 if fixed else None)
    tables = random_tables(lengths, bs, pages, g)
    q = torch.randn(len(lengths), hq, d, generator=g).to(q_dtype)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    if fixed:
        kss, vss = torch.tensor(0.05), torch.tensor(0.02)
        args_dev = (kss.to(dev), vss.to(dev))
        args_cpu = (kss, vss)
    else:
        args_dev = (ks.to(dev)[:, 1], vs.to(dev)[:, 1])
        args_cpu = (ks[:, 1], vs[:, 1])
    got = kernel(q.to(dev), kc.to(dev)[:, 1], vc.to(dev)[:, 1], tables.to(dev), ctx.to(dev), *args_dev)
    want = oatt.paged_attention(q, kc[:, 1], vc[:, 1], tables, ctx, *args_cpu)
    tol = 2e-2 if q_dtype == torch.bfloat16 else 1e-5
    torch.testing.assert_close(got.float().cpu(), want.float(), atol=tol, rtol=tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_sliding_window_matches_oracle(kernel, dev, dtype):
    # reference: kernels/paged_attention.py:50-90; tests/test_fp8_kv_cache.py:87-103
    _say("window", dtype)
    g = torch.Generator().manual_seed(9)
    bs, hkv, hq, d = 16, 4, 8, 128
    lengths = [1, 3, 40, 600, 2000]
    pages = sum(-(-n // bs) for n in lengths)
    _, _, k, v = make_pool(pages, 1, bs, hkv, d, dtype, g)
    tables = random_tables(lengths, bs, pages, g)
    q = torch.randn(len(lengths), hq, d, generator=g).to(dtype)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    for window in (3, 100, 513):
        got = kernel.windowed(q.to(dev), k.to(dev), v.to(dev), tables.to(dev), ctx.to(dev), window)
        _close(got, oatt.paged_attention(q, k, v, tables, ctx, window=window), dtype)


def test_empty_batch_and_bad_arguments(kernel, dev):
    q = torch.empty(0, 4, 128, device=dev, dtype=torch.bfloat16)
    k = torch.zeros(4, 16, 2, 128, device=dev, dtype=torch.bfloat16)
    t = torch.zeros(0, 1, dtype=torch.int32, device=dev)
    out = kernel(q, k, k, t, torch.zeros(0, dtype=torch.int32, device=dev))
    assert out.shape == (0, 4, 128)
    with pytest.raises(ValueError):
        kernel(torch.zeros(1, 3, 128, device=dev, dtype=torch.bfloat16), k, k,
               torch.zeros(1, 1, dtype=torch.int32, device=dev),
               torch.ones(1, dtype=torch.int32, device=dev))
    with pytest.raises(ValueError):
        kernel.windowed(q, k, k, t, t[:, 0], 0)


def test_int32_block_ids_use_64bit_offsets(kernel, dev):
    # reference: tests/test_attention_64bit.py:8-29
    if torch.cuda.mem_get_info()[0] < 9 * 2**30:
        pytest.skip("needs 9 GiB free")
    shape, strides = (2049, 1, 1, 16), (2**20, 16, 16, 1)
    key = torch.empty_strided(shape, strides, device=dev, dtype=torch.float16)
    value = torch.empty_strided(shape, strides, device=dev, dtype=torch.float16)
    key[0].zero_()
    value[0].fill_(-3)
    key[2048].fill_(1)
    expected = torch.arange(16, device=dev, dtype=torch.float16).view(1, 1, 16)
    value[2048].copy_(expected)
    query = torch.ones((1, 1, 16), device=dev, dtype=torch.float16)
    table = torch.tensor([[2048]], device=dev, dtype=torch.int32)
    out = kernel(query, key, value, table, torch.tensor([1], device=dev, dtype=torch.int32))
    torch.cuda.synchronize()
    torch.testing.assert_close(out, expected, rtol=0, atol=0)


def test_out_of_pool_table_entries_stay_inside_the_pool(kernel, dev):
    # A corrupt table entry must not address memory outside the pool (reads block 0).
    k = torch.randn(4, 16, 1, 64, device=dev, dtype=torch.bfloat16)
    q = torch.randn(1, 1, 64, device=dev, dtype=torch.bfloat16)
    bad = torch.tensor([[-1, 1 << 30]], device=dev, dtype=torch.int32)
    good = torch.tensor([[0, 0]], device=dev, dtype=torch.int32)
    ctx = torch.tensor([32], device=dev, dtype=torch.int32)
    assert torch.equal(kernel(q, k, k, bad, ctx), kernel(q, k, k, good, ctx))


# ---------------------------------------------------------------- BASELINE configs
# Shapes of BASELINE.json configs 2-5 at reduced batch (the oracle is a Python loop);
# the full-size configs run in bench.py.

def _plane_tables(n_req, planes, max_len, bs, g, pool_blocks):
    """LAST_EXITED pools: each request owns `planes` tables of ceil(max_len/bs) blocks."""
    per = -(-max_len // bs)
    order = torch.randperm(pool_blocks, generator=g)
    return order[: n_req * planes * per].view(n_req, planes, per).int()


def test_config2_depth_aware_decode(kernel, dev):
    _say("config2")
    g = torch.Generator().manual_seed(2)
    n, planes, bs, h, d, layers = 8, 4, 16, 16, 128, 2
    lengths = torch.randint(512, 4097, (n,), generator=g)
    exit_depth = torch.randint(1, 5, (n,), generator=g)
    pool = n * planes * 256
    kpool, vpool, k, v = make_pool(pool, layers, bs, h, d, torch.bfloat16, g, layer=1)
    tables = _plane_tables(n, planes, 4096, bs, g, pool)
    row_tables = tables[torch.arange(n), exit_depth - 1]
    q = torch.randn(n, h, d, generator=g).bfloat16()
    ctx = lengths.int()
    got = kernel(q.to(dev), kpool.to(dev)[:, 1], vpool.to(dev)[:, 1], row_tables.to(dev), ctx.to(dev))
    _close(got, oatt.paged_attention(q, k, v, row_tables, ctx), torch.bfloat16)


def test_config3_verify_window_gqa4(kernel, dev):
    _say("config3")
    g = torch.Generator().manual_seed(3)
    n, w, bs, hq, hkv, d = 6, 5, 16, 16, 4, 128
    lengths = torch.randint(1024, 8193, (n,), generator=g)
    pool = n * 512
    _, _, k, v = make_pool(pool, 1, bs, hkv, d, torch.bfloat16, g)
    tables = torch.randperm(pool, generator=g)[: n * 512].view(n, 512).int()
    q = torch.randn(n * w, hq, d, generator=g).bfloat16()
    cu = torch.arange(0, n * w + 1, w, dtype=torch.int32)
    got = kernel.prefill(q.to(dev), k.to(dev), v.to(dev), tables.to(dev), lengths.int().to(dev),
                         cu.to(dev), w)
    _close(got, oatt.packed_window_attention(q, k, v, tables, lengths.int(), cu), torch.bfloat16)


def test_config4_wide_heads_d96_32_planes(kernel, dev):
    _say("config4")
    g = torch.Generator().manual_seed(4)
    n, w, planes, bs, h, d = 3, 5, 32, 16, 55, 96
    per = 2048 // bs
    pool = n * planes * per
    _, _, k, v = make_pool(pool, 1, bs, h, d, torch.bfloat16, g)
    tables = _plane_tables(n, planes, 2048, bs, g, pool)
    exit_depth = torch.randint(8, 33, (n,), generator=g)
    seq_tables = tables[torch.arange(n), exit_depth - 1]
    lengths = torch.full((n,), 2048, dtype=torch.int32)
    q = torch.randn(n * w, h, d, generator=g).bfloat16()
    cu = torch.arange(0, n * w + 1, w, dtype=torch.int32)
    got = kernel.prefill(q.to(dev), k.to(dev), v.to(dev), seq_tables.to(dev), lengths.to(dev),
                         cu.to(dev), w)
    _close(got, oatt.packed_window_attention(q, k, v, seq_tables, lengths, cu), torch.bfloat16)


@pytest.mark.parametrize("ctx_lo", [16384, 32760])
def test_config5_fp8_rows_at_different_planes(kernel, dev, ctx_lo):
    """Config 5's rows (fp8 KV, per-tensor scales, window row j at plane (d0 + j) mod 4)
    at both ends of its context range U[16384, 32768]: every 1024-position fp8 chunk up
    to the 32nd is compared with the oracle."""
    _say("config5", ctx_lo)
    g = torch.Generator().manual_seed(5 + ctx_lo)
    n, w, planes, bs, hq, hkv, d = 2, 5, 4, 16, 16, 8, 128
    max_len = ctx_lo + 8
    per = -(-max_len // bs)
    pool = n * planes * per
    x = (torch.randn(pool, 1, bs, hkv, d, generator=g) * 8)
    kc = x.clamp(-448, 448).to(torch.float8_e4m3fn)[:, 0]
    vc = (torch.randn(pool, 1, bs, hkv, d, generator=g) * 8).clamp(-448, 448).to(torch.float8_e4m3fn)[:, 0]
    tables = _plane_tables(n, planes, max_len, bs, g, pool)
    start = torch.randint(ctx_lo, ctx_lo + 4, (n,), generator=g)
    d0 = torch.randint(0, planes, (n,), generator=g)
    rows_t, rows_len = [], []
    for i in range(n):
        for j in range(w):
            rows_t.append(tables[i, (d0[i] + j) % planes])
            rows_len.append(int(start[i]) + j + 1)
    row_tables = torch.stack(rows_t)
    ctx = torch.tensor(rows_len, dtype=torch.int32)
    q = torch.randn(n * w, hq, d, generator=g).bfloat16()
    sk, sv = torch.tensor(0.03), torch.tensor(0.05)
    got = kernel(q.to(dev), kc.to(dev), vc.to(dev), row_tables.to(dev), ctx.to(dev), sk.to(dev), sv.to(dev))
    _close(got, oatt.paged_attention(q, kc, vc, row_tables, ctx, sk, sv), torch.bfloat16)


def test_large_batch_rows_equal_single_row_launches_bitwise(kernel, dev):
    # A batch's units are spread over persistent per-CU workgroups; a row's result
    # must not depend on which workgroup or wave served it.
    _say("persistent assignment")
    g = torch.Generator().manual_seed(11)
    bs, hq, hkv, d, dtype = 16, 16, 4, 128, torch.bfloat16
    lengths = torch.randint(1, 8193, (16,), generator=g).tolist()
    lengths[0], lengths[1] = 8192, 513
    width = 8192 // bs
    pages = sum(-(-n // bs) for n in lengths)
    _, _, k, v = make_pool(pages, 1, bs, hkv, d, dtype, g)
    tables = random_tables(lengths, bs, pages, g, width=width)
    q = torch.randn(len(lengths), hq, d, generator=g).to(dtype)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    kd, vd, td, cd, qd = k.to(dev), v.to(dev), tables.to(dev), ctx.to(dev), q.to(dev)
    got = kernel(qd, kd, vd, td, cd)
    for row in (0, 1, 7):
        alone = kernel(qd[row:row + 1], kd, vd, td[row:row + 1], cd[row:row + 1])
        assert torch.equal(alone[0], got[row])
    sel = [0, 1, 7]
    want = oatt.paged_attention(q[sel], k, v, tables[sel], ctx[sel])
    _close(got[sel], want, dtype)


def test_more_rows_than_the_persistent_index_uses_grid_kernel(kernel, dev):
    # More than 8192 (sequence, row-group) pairs run one single-wave workgroup per
    # unit; same per-unit arithmetic as the persistent kernel.
    _say("grid fallback")
    g = torch.Generator().manual_seed(12)
    bs, hq, hkv, d, dtype = 16, 2, 1, 64, torch.bfloat16
    n = 8200
    lengths = torch.randint(0, 41, (n,), generator=g).tolist()
    pages = sum(-(-x // bs) for x in lengths)
    _, _, k, v = make_pool(pages, 1, bs, hkv, d, dtype, g)
    tables = random_tables(lengths, bs, pages, g)
    q = torch.randn(n, hq, d, generator=g).to(dtype)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    kd, vd, td, cd, qd = k.to(dev), v.to(dev), tables.to(dev), ctx.to(dev), q.to(dev)
    got = kernel(qd, kd, vd, td, cd)
    sel = [0, 1, 4097, 8199] + [i for i in range(n) if lengths[i] == 0][:1]
    for row in sel:
        alone = kernel(qd[row:row + 1], kd, vd, td[row:row + 1], cd[row:row + 1])
        assert torch.equal(alone[0], got[row])
    want = oatt.paged_attention(q[sel], k, v, tables[sel], ctx[sel])
    _close(got[sel], want, dtype)


def _dense_packed(q, k_seq, v_seq, q_len, length, window=0):
    """Closed form: fp32 SDPA of one sequence's q_len queries over its `length` keys,
    query i at absolute position length - q_len + i (bottom-right causal), seeing the
    last `window` keys when window > 0; GQA by kv head h // (Hq / Hkv)."""
    hq, hkv = q.shape[1], k_seq.shape[1]
    kk = k_seq.float().repeat_interleave(hq // hkv, 1).transpose(0, 1)
    vv = v_seq.float().repeat_interleave(hq // hkv, 1).transpose(0, 1)
    pos = torch.arange(length - q_len, length).view(-1, 1)
    key = torch.arange(length).view(1, -1)
    mask = key <= pos
    if window:
        mask &= key > pos - window
    return torch.nn.functional.scaled_dot_product_attention(
        q.float().transpose(0, 1), kk, vv, attn_mask=mask[None]).transpose(0, 1)


@pytest.mark.parametrize("window", [0, 256])
@pytest.mark.parametrize("dtype,d,hq,hkv", [(torch.bfloat16, 128, 16, 4),
                                            (torch.float16, 64, 8, 8),
                                            (torch.bfloat16, 64, 4, 1),
                                            (torch.float16, 128, 6, 2),
                                            (torch.bfloat16, 96, 8, 2)])
def test_long_prompt_prefill_matches_dense_causal(kernel, dev, window, dtype, d, hq, hkv):
    """Prompt prefill on the same backend: a 1024-token prompt from scratch, a
    512-token chunk after a 1536-token prefix, ragged windows (64, 97 and 129 rows,
    one shorter than its 128-row group), and a short window, packed together."""
    _say("long prefill", window, dtype, d, hq, hkv)
    g = torch.Generator().manual_seed(21)
    bs = 16
    seqs = [(1024, 1024), (2048, 512), (3000, 37), (64, 64), (300, 97), (129, 129)]
    pages = sum(-(-n // bs) for n, _ in seqs) + 2
    _, _, k, v = make_pool(pages, 1, bs, hkv, d, dtype, g)
    tables = random_tables([n for n, _ in seqs], bs, pages, g)
    total = sum(c for _, c in seqs)
    q = torch.randn(total, hq, d, generator=g).to(dtype)
    lengths = torch.tensor([n for n, _ in seqs], dtype=torch.int32)
    cu = torch.tensor([0] + list(torch.tensor([c for _, c in seqs]).cumsum(0)), dtype=torch.int32)
    got = kernel.prefill(q.to(dev), k.to(dev), v.to(dev), tables.to(dev), lengths.to(dev),
                         cu.to(dev), max(c for _, c in seqs), window=window).cpu()
    for s, (n, c) in enumerate(seqs):
        pages_s = tables[s, : -(-n // bs)].long()
        k_seq = k[pages_s].reshape(-1, hkv, d)[:n]
        v_seq = v[pages_s].reshape(-1, hkv, d)[:n]
        want = _dense_packed(q[cu[s]:cu[s + 1]], k_seq, v_seq, c, n, window)
        torch.testing.assert_close(got[cu[s]:cu[s + 1]].float(), want, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("window", [0, 256])
@pytest.mark.parametrize("per_vector", [False, True])
@pytest.mark.parametrize("q_dtype,d,hq,hkv,bs", [(torch.bfloat16, 128, 16, 8, 16),
                                                 (torch.float16, 96, 8, 2, 16),
                                                 (torch.bfloat16, 64, 8, 8, 8)])
def test_long_prompt_prefill_fp8_matches_dense_causal(kernel, dev, per_vector, q_dtype, d, hq,
                                                      hkv, bs, window):
    """Prompt prefill over an FP8 pool (reference: triton_attention.py:335-362,460-487,
    the packed kernel's HAS_SCALE loads): long prompts, a chunk after a prefix and ragged
    windows against dense causal SDPA over the dequantized keys and values, with
    per-tensor or per-vector scales.  These windows take the prefill tiling (fp8 tiles
    widened to q's type in LDS, head_dim 96 on 128-dim LDS rows)."""
    _say("long prefill fp8", per_vector, q_dtype, d, bs, window)
    g = torch.Generator().manual_seed(23 + d)
    assert kernel.uses_prefill_tiling(q_dtype, torch.float8_e4m3fn, d, 1024)
    seqs = [(1024, 1024), (2048, 512), (3000, 37), (300, 97), (129, 129)]
    pages = sum(-(-n // bs) for n, _ in seqs) + 2
    x_k = torch.randn(pages, bs, hkv, d, generator=g) * 3
    x_v = torch.randn(pages, bs, hkv, d, generator=g) * 3
    if per_vector:
        kc, ks = ofp8.quantize_fp8(x_k)
        vc, vs = ofp8.quantize_fp8(x_v)
        k_deq, v_deq = ofp8.dequantize_fp8(kc, ks, torch.float32), ofp8.dequantize_fp8(vc, vs, torch.float32)
        sk, sv = ks.to(dev), vs.to(dev)
    else:
        kc, ks = ofp8.quantize_fp8(x_k, 0.02)
        vc, vs = ofp8.quantize_fp8(x_v, 0.03)
        k_deq, v_deq = kc.float() * 0.02, vc.float() * 0.03
        sk, sv = torch.tensor(0.02, device=dev), torch.tensor(0.03, device=dev)
    tables = random_tables([n for n, _ in seqs], bs, pages, g)
    total = sum(c for _, c in seqs)
    q = torch.randn(total, hq, d, generator=g).to(q_dtype)
    lengths = torch.tensor([n for n, _ in seqs], dtype=torch.int32)
    cu = torch.tensor([0] + list(torch.tensor([c for _, c in seqs]).cumsum(0)), dtype=torch.int32)
    got = kernel.prefill(q.to(dev), kc.to(dev), vc.to(dev), tables.to(dev), lengths.to(dev),
                         cu.to(dev), max(c for _, c in seqs), sk, sv, window=window).cpu()
    for s, (n, c) in enumerate(seqs):
        pages_s = tables[s, : -(-n // bs)].long()
        k_seq = k_deq[pages_s].reshape(-1, hkv, d)[:n]
        v_seq = v_deq[pages_s].reshape(-1, hkv, d)[:n]
        want = _dense_packed(q[cu[s]:cu[s + 1]], k_seq, v_seq, c, n, window)
        torch.testing.assert_close(got[cu[s]:cu[s + 1]].float(), want, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("bs,window,dtype,d", [(8, 0, torch.bfloat16, 128),
                                               (8, 256, torch.bfloat16, 128),
                                               (48, 0, torch.bfloat16, 128),
                                               (32, 100, torch.bfloat16, 128),
                                               (8, 0, torch.float16, 64),
                                               (32, 300, torch.float16, 64),
                                               (8, 0, torch.bfloat16, 96),
                                               (32, 100, torch.float16, 96)])
def test_long_prompt_prefill_block_sizes(kernel, dev, bs, window, dtype, d):
    """The prefill tiling's two address paths: blocks holding whole 16-position groups
    (one table lookup per group, 32 and 48 here) and smaller blocks (a lookup per
    position, 8 here), with and without a sliding window, at head_dim 128 and 64 (the
    direct loads fill 4 and 8 rows per instruction) and 96 (128-dim LDS rows whose pad
    slots no lane loads)."""
    _say("long prefill block size", bs, window, dtype, d)
    g = torch.Generator().manual_seed(22)
    hq, hkv = 16, 4
    seqs = [(1024, 1024), (2000, 700), (129, 129)]
    pages = sum(-(-n // bs) for n, _ in seqs) + 2
    _, _, k, v = make_pool(pages, 1, bs, hkv, d, dtype, g)
    tables = random_tables([n for n, _ in seqs], bs, pages, g)
    total = sum(c for _, c in seqs)
    q = torch.randn(total, hq, d, generator=g).to(dtype)
    lengths = torch.tensor([n for n, _ in seqs], dtype=torch.int32)
    cu = torch.tensor([0] + list(torch.tensor([c for _, c in seqs]).cumsum(0)), dtype=torch.int32)
    got = kernel.prefill(q.to(dev), k.to(dev), v.to(dev), tables.to(dev), lengths.to(dev),
                         cu.to(dev), max(c for _, c in seqs), window=window).cpu()
    for s, (n, c) in enumerate(seqs):
        pages_s = tables[s, : -(-n // bs)].long()
        k_seq = k[pages_s].reshape(-1, hkv, d)[:n]
        v_seq = v[pages_s].reshape(-1, hkv, d)[:n]
        want = _dense_packed(q[cu[s]:cu[s + 1]], k_seq, v_seq, c, n, window)
        torch.testing.assert_close(got[cu[s]:cu[s + 1]].float(), want, atol=2e-2, rtol=2e-2)


# ------------------------------------------ packed rows with explicit row lengths

def _group_rows_by_plane(n, w, planes, d0, row_len, order="ascending"):
    """Pipelined verify rows: row j of request i reads plane (d0[i] + j) % planes.  One
    packed sequence per (request, plane), its rows by length (``order`` ascending or
    descending) or in a mixed order (``rotated``: the longest row first)."""
    perm, cu, seq_req, seq_plane = [], [0], [], []
    for i in range(n):
        for pl in range(planes):
            rows = [i * w + j for j in range(w) if (int(d0[i]) + j) % planes == pl]
            if not rows:
                continue
            rows.sort(key=lambda r: int(row_len[r]), reverse=order == "descending")
            if order == "rotated":
                rows = rows[-1:] + rows[:-1]
            perm += rows
            cu.append(len(perm))
            seq_req.append(i)
            seq_plane.append(pl)
    return (torch.tensor(perm), torch.tensor(cu, dtype=torch.int32), torch.tensor(seq_req),
            torch.tensor(seq_plane))


@pytest.mark.parametrize("q_dtype,kv,planes,hq,hkv,d,window,order", [
    (torch.bfloat16, "fp8", 4, 16, 8, 128, 0, "ascending"),   # config 5: rows 0 and 4 share d0
    (torch.bfloat16, "bf16", 2, 16, 2, 128, 0, "ascending"),  # 3 rows x GQA 8: two row tiles
    (torch.float16, "fp16", 4, 8, 8, 64, 300, "ascending"),   # windowed
    (torch.float32, "fp32", 3, 4, 2, 32, 0, "ascending"),     # vector path
    # rows of a sequence in any order (each unit bounds over all of its rows)
    (torch.bfloat16, "fp8", 4, 16, 8, 128, 0, "descending"),
    (torch.bfloat16, "bf16", 2, 16, 2, 128, 0, "rotated"),
    (torch.float16, "fp16", 4, 8, 8, 64, 300, "descending"),
    (torch.float32, "fp32", 3, 4, 2, 32, 0, "rotated"),
])
def test_packed_rows_with_row_lengths_equal_per_row_bitwise(kernel, dev, q_dtype, kv, planes, hq,
                                                            hkv, d, window, order):
    _say("row_lengths", q_dtype, kv, planes, hq, hkv, d, window, order)
    g = torch.Generator().manual_seed(11)
    n, w, bs = 5, 5, 16
    max_len = 3000 + w
    per = -(-max_len // bs)
    pool = n * planes * per
    if kv == "fp8":
        kc = (torch.randn(pool, bs, hkv, d, generator=g) * 8).to(torch.float8_e4m3fn)
        vc = (torch.randn(pool, bs, hkv, d, generator=g) * 8).to(torch.float8_e4m3fn)
        sk, sv = torch.tensor(0.03), torch.tensor(0.05)
    else:
        kv_dtype = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[kv]
        kc = torch.randn(pool, bs, hkv, d, generator=g).to(kv_dtype)
        vc = torch.randn(pool, bs, hkv, d, generator=g).to(kv_dtype)
        sk = sv = None
    tables = torch.randperm(pool, generator=g)[: n * planes * per].view(n, planes, per).int()
    start = torch.randint(1, 3000, (n,), generator=g)
    start[0] = 507  # the window straddles a 512-position chunk boundary
    d0 = torch.randint(0, planes, (n,), generator=g)
    j = torch.arange(w)
    plane = (d0.view(n, 1) + j.view(1, w)) % planes
    row_tables = tables[torch.arange(n).view(n, 1), plane].reshape(n * w, per)
    row_len = (start.view(n, 1) + j.view(1, w) + 1).reshape(-1).int()
    q = torch.randn(n * w, hq, d, generator=g).to(q_dtype)
    perm, cu, seq_req, seq_plane = _group_rows_by_plane(n, w, planes, d0, row_len, order)
    seq_tables = tables[seq_req, seq_plane]
    seq_len = torch.stack([row_len[perm[cu[s]:cu[s + 1]]].max() for s in range(len(cu) - 1)])
    max_q = int((cu[1:] - cu[:-1]).max())
    kd, vd = kc.to(dev), vc.to(dev)
    skd = sk.to(dev) if sk is not None else None
    svd = sv.to(dev) if sv is not None else None
    if window:
        per_row = kernel.windowed(q.to(dev), kd, vd, row_tables.to(dev), row_len.to(dev), window,
                                  skd, svd)
    else:
        per_row = kernel(q.to(dev), kd, vd, row_tables.to(dev), row_len.to(dev), skd, svd)
    packed = kernel.prefill(q[perm].contiguous().to(dev), kd, vd, seq_tables.to(dev),
                            seq_len.int().to(dev), cu.to(dev), max_q, skd, svd, window=window,
                            row_lengths=row_len[perm].to(dev))
    assert torch.equal(packed.cpu(), per_row.cpu()[perm])
    if window:
        want = oatt.paged_attention(q, kc, vc, row_tables, row_len, sk, sv, window)
    else:
        want = oatt.paged_attention(q, kc, vc, row_tables, row_len, sk, sv)
    _close(packed.cpu(), want[perm], q_dtype)


def test_row_lengths_need_the_packed_form(kernel, dev):
    q = torch.zeros(2, 4, 64, device=dev, dtype=torch.bfloat16)
    k = torch.zeros(4, 16, 4, 64, device=dev, dtype=torch.bfloat16)
    t = torch.zeros(2, 2, device=dev, dtype=torch.int32)
    ln = torch.full((2,), 8, device=dev, dtype=torch.int32)
    with pytest.raises(ValueError):
        kernel._run(q, k, k, t, ln, None, 1, None, None, 0, ln)
    cu = torch.tensor([0, 2], device=dev, dtype=torch.int32)
    with pytest.raises(ValueError):
        kernel.prefill(q, k, k, t[:1], ln[:1], cu, 2, row_lengths=ln[:1])


def test_row_lengths_on_the_grid_kernel(kernel, dev):
    # 8200 packed sequences of two rows (more than 8192 pairs: the grid kernel); row 0
    # of each sequence sees a key count a few positions below row 1's, as pipelined
    # rows on one plane do.  Every row equals its per-row launch bit for bit.
    _say("row_lengths grid kernel")
    g = torch.Generator().manual_seed(13)
    bs, hq, hkv, d, dtype = 16, 2, 1, 64, torch.bfloat16
    n = 8200
    hi = torch.randint(5, 41, (n,), generator=g)
    lo = hi - torch.randint(0, 5, (n,), generator=g)
    lengths = hi.tolist()
    pages = sum(-(-x // bs) for x in lengths)
    _, _, k, v = make_pool(pages, 1, bs, hkv, d, dtype, g)
    tables = random_tables(lengths, bs, pages, g)
    q = torch.randn(2 * n, hq, d, generator=g).to(dtype)
    row_len = torch.stack([lo, hi], 1).reshape(-1).int()
    row_tables = tables.repeat_interleave(2, 0)
    cu = torch.arange(0, 2 * n + 1, 2, dtype=torch.int32)
    kd, vd, qd = k.to(dev), v.to(dev), q.to(dev)
    got = kernel.prefill(qd, kd, vd, tables.to(dev), hi.int().to(dev), cu.to(dev), 2,
                         row_lengths=row_len.to(dev))
    per_row = kernel(qd, kd, vd, row_tables.to(dev), row_len.to(dev))
    assert torch.equal(got, per_row)
    sel = [0, 1, 8198, 16399]
    want = oatt.paged_attention(q[sel], k, v, row_tables[sel], row_len[sel])
    _close(got[sel].cpu(), want, dtype)


# ------------------------------------------------------------ window store + attention

def _window_store_case(g, dtype, d, hq, hkv, bs, lengths, q_lens, pool_blocks, layers=2,
                       layer=1):
    kpool, vpool, _, _ = make_pool(pool_blocks, layers, bs, hkv, d, dtype, g)
    tables = random_tables(lengths, bs, pool_blocks, g)
    rows = sum(q_lens)
    q = torch.randn(rows, hq, d, generator=g).to(dtype)
    k_new = torch.randn(rows, hkv, d, generator=g).to(dtype)
    v_new = torch.randn(rows, hkv, d, generator=g).to(dtype)
    cu = torch.tensor([0] + list(torch.tensor(q_lens).cumsum(0)), dtype=torch.int32)
    return kpool, vpool, tables, q, k_new, v_new, cu


@pytest.mark.parametrize("long_window", [False, True])
@pytest.mark.parametrize("dtype,d,hq,hkv,bs", [
    (torch.bfloat16, 128, 16, 4, 16),   # config 3's heads
    (torch.float16, 64, 8, 8, 16),
    (torch.bfloat16, 96, 4, 1, 16),
    (torch.bfloat16, 128, 8, 2, 5),     # blocks that do not hold whole tiles
])
def test_prefill_store_equals_store_then_prefill(kernel, pkg, dev, dtype, d, hq, hkv, bs,
                                                 long_window):
    """The fused window store + attention writes the pool and returns the output of
    store_kv at the window positions followed by prefill, bit for bit.  Windows sit on
    both sides of the 256-position half-chunk and 512-position chunk boundaries, and a
    9-row window over GQA 4 spans two row groups (two units write the same positions).
    With long windows (the longest 130 rows) the call takes the prefill tiling and stores
    with the window-store kernel first."""
    _say("prefill_store", dtype, d, hq, hkv, bs, long_window)
    g = torch.Generator().manual_seed(d + hq + bs + long_window)
    lengths = [5, 258, 514, 1030, 3000, 9, 40, 1]
    q_lens = [5, 5, 5, 9, 1, 9, 33, 1]
    if long_window:
        lengths = [70, 300, 1030, 2000, 129, 64, 5]
        q_lens = [70, 65, 130, 64, 129, 64, 5]
    assert kernel.uses_prefill_tiling(dtype, dtype, d, max(q_lens)) == long_window
    pages = sum(-(-x // bs) for x in lengths) + 7
    kpool, vpool, tables, q, k_new, v_new, cu = _window_store_case(
        g, dtype, d, hq, hkv, bs, lengths, q_lens, pages)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    max_q = max(q_lens)
    # separate: store_kv at the window positions, then prefill
    ka, va = kpool.to(dev), vpool.to(dev)
    seq = torch.repeat_interleave(torch.arange(len(q_lens)), torch.tensor(q_lens))
    pos = ctx.long()[seq] - torch.tensor(q_lens)[seq] + torch.arange(len(seq)) - cu.long()[seq]
    blocks = tables.long()[seq, pos // bs]
    pkg.store_kv(ka[:, 1], va[:, 1], k_new.to(dev), v_new.to(dev), blocks.to(dev),
                 (pos % bs).to(dev))
    want = kernel.prefill(q.to(dev), ka[:, 1], va[:, 1], tables.to(dev), ctx.to(dev),
                          cu.to(dev), max_q)
    # fused
    kb, vb = kpool.to(dev), vpool.to(dev)
    got = kernel.prefill_store(q.to(dev), k_new.to(dev), v_new.to(dev), kb[:, 1], vb[:, 1],
                               tables.to(dev), ctx.to(dev), cu.to(dev), max_q)
    assert torch.equal(kb.view(torch.int16), ka.view(torch.int16))
    assert torch.equal(vb.view(torch.int16), va.view(torch.int16))
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # the other layer of the pool is untouched
    assert torch.equal(kb[:, 0].cpu().view(torch.int16), kpool[:, 0].view(torch.int16))


def test_prefill_store_graph_replays_and_other_shapes(kernel, pkg, dev):
    """Replayed from a HIP graph the fused form gives the eager result every time (the
    pool is rewritten with the same rows); shapes it does not serve -- float32 q, a
    prefill-length window -- store and attend separately with the same result; a table
    entry outside the pool writes nothing."""
    _say("prefill_store graph / fallbacks")
    g = torch.Generator().manual_seed(77)
    bs, hq, hkv, d = 16, 16, 4, 128
    lengths, q_lens = [700, 1500, 64, 2049], [5, 5, 64, 5]
    pages = sum(-(-x // bs) for x in lengths) + 3
    kpool, vpool, tables, q, k_new, v_new, cu = _window_store_case(
        g, torch.bfloat16, d, hq, hkv, bs, lengths, q_lens, pages, layers=1, layer=0)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    args = lambda kp, vp, qq: (qq, k_new.to(dev), v_new.to(dev), kp[:, 0], vp[:, 0],
                               tables.to(dev), ctx.to(dev), cu.to(dev), max(q_lens))
    # q_len 64 takes the prefill tiling: a separate store, then attention
    seq = torch.repeat_interleave(torch.arange(4), torch.tensor(q_lens))
    pos = ctx.long()[seq] - torch.tensor(q_lens)[seq] + torch.arange(len(seq)) - cu.long()[seq]
    ks, vs = kpool.to(dev), vpool.to(dev)
    pkg.store_kv(ks[:, 0], vs[:, 0], k_new.to(dev), v_new.to(dev),
                 tables.long()[seq, pos // bs].to(dev), (pos % bs).to(dev))
    ka, va = kpool.to(dev), vpool.to(dev)
    got64 = kernel.prefill_store(*args(ka, va, q.to(dev)))
    assert torch.equal(ka.view(torch.int16), ks.view(torch.int16))
    assert torch.equal(va.view(torch.int16), vs.view(torch.int16))
    want64 = kernel.prefill(q.to(dev), ks[:, 0], vs[:, 0], tables.to(dev), ctx.to(dev),
                            cu.to(dev), 64)
    assert torch.equal(got64.view(torch.int16), want64.view(torch.int16))
    # three 5-row windows: the fused form, bitwise the separate store + verify kernels
    sel = [0, 1, 3]
    rows = torch.cat([torch.arange(cu[s], cu[s + 1]) for s in sel])
    cu3 = torch.tensor([0, 5, 10, 15], dtype=torch.int32)
    kb, vb = kpool.to(dev), vpool.to(dev)
    qd, kn, vn = q[rows].to(dev), k_new[rows].to(dev), v_new[rows].to(dev)
    t3, c3 = tables[sel].to(dev), ctx[sel].to(dev)
    eager = kernel.prefill_store(qd, kn, vn, kb[:, 0], vb[:, 0], t3, c3, cu3.to(dev), 5)
    want = kernel.prefill(qd, ks[:, 0], vs[:, 0], t3, c3, cu3.to(dev), 5)
    assert torch.equal(eager.view(torch.int16), want.view(torch.int16))
    stream = torch.cuda.Stream()
    cu3d = cu3.to(dev)
    with torch.cuda.stream(stream):
        kernel.prefill_store(qd, kn, vn, kb[:, 0], vb[:, 0], t3, c3, cu3d, 5)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = kernel.prefill_store(qd, kn, vn, kb[:, 0], vb[:, 0], t3, c3, cu3d, 5)
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
        torch.cuda.synchronize()
    # float32 q: the vector kernels, separate store
    kc, vc = kpool.to(dev), vpool.to(dev)
    got32 = kernel.prefill_store(qd.float(), kn, vn, kc[:, 0], vc[:, 0], t3, c3, cu3.to(dev), 5)
    assert torch.equal(kc.view(torch.int16), kb.view(torch.int16))
    ref32 = kernel.prefill(qd.float(), kb[:, 0], vb[:, 0], t3, c3, cu3.to(dev), 5)
    assert torch.equal(got32, ref32)
    # a table entry outside the pool: that window position is not written
    bad = t3.clone()
    last = (c3[0].item() - 1) // bs
    bad[0, last] = pages + 5
    kd, vd = kpool.to(dev), vpool.to(dev)
    kernel.prefill_store(qd, kn, vn, kd[:, 0], vd[:, 0], bad, c3, cu3.to(dev), 5)
    blk = t3[0, last].item()
    assert torch.equal(kd[blk].cpu().view(torch.int16), kpool[blk].view(torch.int16))


@pytest.mark.parametrize("form", ["fused", "prefill_tiling", "float32_q"])
def test_prefill_store_skips_positions_outside_the_table_or_pool(kernel, pkg, dev, form):
    """Every form of prefill_store (the one-launch form, the window-store kernel ahead of
    the prefill tiling, and the separate store of float32 q) leaves unwritten a window
    position whose block index lies beyond the table width or whose table entry lies
    outside the pool, and writes every other window position."""
    _say("prefill_store outside", form)
    g = torch.Generator().manual_seed(91)
    bs, hq, hkv, d = 16, 8, 2, 128
    q_len = 64 if form == "prefill_tiling" else 5
    lengths = [700, 2049, 300]
    pages = sum(-(-x // bs) for x in lengths) + 3
    kpool, vpool, tables, q, k_new, v_new, cu = _window_store_case(
        g, torch.bfloat16, d, hq, hkv, bs, lengths, [q_len] * 3, pages, layers=1, layer=0)
    width = -(-2049 // bs) - 1  # position 2048 of sequence 1 lies beyond the table
    tables = tables[:, :width]
    tables[0, (700 - 1) // bs] = pages + 5  # sequence 0's last block: outside the pool
    ctx = torch.tensor(lengths, dtype=torch.int32)
    if form == "float32_q":
        q = q.float()
    kd, vd = kpool.to(dev), vpool.to(dev)
    kernel.prefill_store(q.to(dev), k_new.to(dev), v_new.to(dev), kd[:, 0], vd[:, 0],
                         tables.to(dev), ctx.to(dev), cu.to(dev), q_len)
    torch.cuda.synchronize()
    ke, ve = kpool.clone(), vpool.clone()
    written = 0
    for s_ in range(3):
        for i in range(q_len):
            pos = lengths[s_] - q_len + i
            idx = pos // bs
            if idx >= width:
                continue
            e = int(tables[s_, idx])
            if not 0 <= e < pages:
                continue
            r = s_ * q_len + i
            ke[e, 0, pos % bs], ve[e, 0, pos % bs] = k_new[r], v_new[r]
            written += 1
    assert 0 < written < 3 * q_len
    assert torch.equal(kd.cpu().view(torch.int16), ke.view(torch.int16))
    assert torch.equal(vd.cpu().view(torch.int16), ve.view(torch.int16))


@pytest.mark.parametrize("per_vector", [False, True])
def test_fp8_prefill_store_long_window_skips_positions_outside(kernel, pkg, dev, per_vector):
    """The window-store kernel ahead of the prefill tiling on an FP8 pool: positions beyond
    the table or in blocks outside the pool keep their codes (and scales); every other
    window position holds the quantize_fp8 codes (and, per vector, scales) of its row."""
    _say("fp8 long-window store outside", per_vector)
    g = torch.Generator().manual_seed(92 + per_vector)
    bs, hq, hkv, d, w = 16, 8, 2, 128, 64
    lengths = [700, 2049, 300]
    n = len(lengths)
    pages = sum(-(-x // bs) for x in lengths) + 3
    kc, vc, ks, vs, tables, q, k_new, v_new = _fp8_store_case(
        g, n, w, hq, hkv, d, bs, lengths, pages, per_vector, torch.bfloat16)
    assert kernel.uses_prefill_tiling(torch.bfloat16, torch.float8_e4m3fn, d, w)
    width = -(-2049 // bs) - 1
    tables = tables[:, :width].contiguous()
    tables[0, (700 - 1) // bs] = pages + 5
    ctx = torch.tensor(lengths, dtype=torch.int32)
    cu = torch.arange(0, n * w + 1, w, dtype=torch.int32)
    kd, vd, ksd, vsd = kc.to(dev), vc.to(dev), ks.to(dev), vs.to(dev)
    fixed = 0.05
    if per_vector:
        kernel.prefill_store(q.to(dev), k_new.to(dev), v_new.to(dev), kd, vd, tables.to(dev),
                             ctx.to(dev), cu.to(dev), w, ksd, vsd)
    else:
        s0 = torch.tensor(fixed, device=dev)
        kernel.prefill_store(q.to(dev), k_new.to(dev), v_new.to(dev), kd, vd, tables.to(dev),
                             ctx.to(dev), cu.to(dev), w, s0, s0)
    torch.cuda.synchronize()
    ke, ve, kse, vse = kc.clone(), vc.clone(), ks.clone(), vs.clone()
    kq, kqs = ofp8.quantize_fp8(k_new.float(), None if per_vector else fixed)
    vq, vqs = ofp8.quantize_fp8(v_new.float(), None if per_vector else fixed)
    written = 0
    for s_ in range(n):
        for i in range(w):
            pos = lengths[s_] - w + i
            idx = pos // bs
            if idx >= width:
                continue
            e = int(tables[s_, idx])
            if not 0 <= e < pages:
                continue
            r = s_ * w + i
            ke[e, pos % bs], ve[e, pos % bs] = kq[r], vq[r]
            if per_vector:
                kse[e, pos % bs], vse[e, pos % bs] = kqs[r], vqs[r]
            written += 1
    assert 0 < written < n * w
    assert torch.equal(kd.cpu().view(torch.uint8), ke.view(torch.uint8))
    assert torch.equal(vd.cpu().view(torch.uint8), ve.view(torch.uint8))
    assert torch.equal(ksd.cpu(), kse) and torch.equal(vsd.cpu(), vse)


# ------------------------------------------------------------ FP8 window store + attention

def _fp8_store_case(g, n, w, hq, hkv, d, bs, lengths, pool_blocks, per_vector, q_dtype):
    """FP8 pools (codes, per-vector scales), tables and a window of w rows per sequence."""
    x = torch.randn(pool_blocks, bs, hkv, d, generator=g) * 3
    kc, ks = ofp8.quantize_fp8(x)
    vc, vs = ofp8.quantize_fp8(torch.randn(pool_blocks, bs, hkv, d, generator=g) * 3)
    tables = random_tables(lengths, bs, pool_blocks, g)
    q = torch.randn(n * w, hq, d, generator=g).to(q_dtype)
    k_new = (torch.randn(n * w, hkv, d, generator=g) * 4).to(q_dtype)
    v_new = (torch.randn(n * w, hkv, d, generator=g) * 4).to(q_dtype)
    k_new[0, 0, 3] = 0.0  # a zero vector component and a fully zero vector (tiny scale)
    v_new[1, 0].zero_()
    return kc, vc, ks, vs, tables, q, k_new, v_new


@pytest.mark.parametrize("w", [5, 70])
@pytest.mark.parametrize("per_vector", [False, True])
@pytest.mark.parametrize("q_dtype,d,hq,hkv", [(torch.bfloat16, 128, 16, 8),
                                              (torch.float16, 96, 4, 2)])
def test_fp8_prefill_store_equals_store_fp8_then_prefill(kernel, pkg, dev, per_vector, q_dtype, d,
                                                         hq, hkv, w):
    """The FP8 window store fused with the attention launch (a 5-row window; a 70-row one
    stores with the window-store kernel ahead of the prefill tiling) writes the codes
    (and, with per-vector scales, the scales) that store_fp8 writes -- bitwise the
    reference's quantize_fp8 -- and returns the attention of prefill over that pool, bit
    for bit.  Per-tensor scales are read, never written."""
    _say("fp8 prefill_store", per_vector, q_dtype, d, w)
    g = torch.Generator().manual_seed(d + hq + per_vector + w)
    bs = 16
    assert kernel.uses_prefill_tiling(q_dtype, torch.float8_e4m3fn, d, w) == (w >= 64)
    lengths = [w, 300, 1030, 1500, 2049]
    n = len(lengths)
    pages = sum(-(-x // bs) for x in lengths) + 5
    kc, vc, ks, vs, tables, q, k_new, v_new = _fp8_store_case(
        g, n, w, hq, hkv, d, bs, lengths, pages, per_vector, q_dtype)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    cu = torch.arange(0, n * w + 1, w, dtype=torch.int32)
    seq = torch.arange(n).repeat_interleave(w)
    pos = ctx.long()[seq] - w + torch.arange(n * w) % w
    blocks, offs = tables.long()[seq, pos // bs], pos % bs
    fixed = 0.0375
    # separate: store_fp8, then prefill
    ka, va, ksa, vsa = kc.to(dev), vc.to(dev), ks.to(dev), vs.to(dev)
    pkg.store_fp8(k_new.to(dev), v_new.to(dev), ka, va, ksa, vsa, blocks.to(dev), offs.to(dev),
                  448.0, fixed_scale=None if per_vector else fixed)
    if per_vector:
        want = kernel.prefill(q.to(dev), ka, va, tables.to(dev), ctx.to(dev), cu.to(dev), w, ksa, vsa)
    else:
        s0 = torch.tensor(fixed, device=dev)
        want = kernel.prefill(q.to(dev), ka, va, tables.to(dev), ctx.to(dev), cu.to(dev), w, s0, s0)
    # fused
    kb, vb, ksb, vsb = kc.to(dev), vc.to(dev), ks.to(dev), vs.to(dev)
    if per_vector:
        got = kernel.prefill_store(q.to(dev), k_new.to(dev), v_new.to(dev), kb, vb, tables.to(dev),
                                   ctx.to(dev), cu.to(dev), w, ksb, vsb)
        assert torch.equal(ksb, ksa) and torch.equal(vsb, vsa)
    else:
        s0 = torch.tensor(fixed, device=dev)
        got = kernel.prefill_store(q.to(dev), k_new.to(dev), v_new.to(dev), kb, vb, tables.to(dev),
                                   ctx.to(dev), cu.to(dev), w, s0, s0)
        assert float(s0) == float(torch.tensor(fixed))  # read, not written
    assert torch.equal(kb.view(torch.uint8), ka.view(torch.uint8))
    assert torch.equal(vb.view(torch.uint8), va.view(torch.uint8))
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # the stored codes are the oracle's quantization of the rows at their positions
    ke = kc.clone()
    codes, _ = ofp8.quantize_fp8(k_new.float(), None if per_vector else fixed)
    ke[blocks, offs] = codes
    assert torch.equal(kb.cpu().view(torch.uint8), ke.view(torch.uint8))


def test_fp8_prefill_store_with_row_lengths_config5_layout(kernel, pkg, dev):
    """Config 5's packed pipeline rows (window row j at plane (d0 + j) mod 4, sequences
    per (request, plane) with explicit row lengths): every row's K / V is quantized into
    its own plane at position row_lengths - 1 and the attention equals store_fp8
    followed by the row-lengths prefill, bit for bit; per-tensor scales; also from a
    replayed HIP graph."""
    _say("fp8 prefill_store row lengths")
    g = torch.Generator().manual_seed(55)
    n, w, planes, bs, hq, hkv, d = 3, 5, 4, 16, 16, 8, 128
    max_len = 3000
    per = -(-max_len // bs)
    pool = n * planes * per
    kc, _ = ofp8.quantize_fp8(torch.randn(pool, bs, hkv, d, generator=g) * 3)
    vc, _ = ofp8.quantize_fp8(torch.randn(pool, bs, hkv, d, generator=g) * 3)
    tables = torch.randperm(pool, generator=g)[: n * planes * per].view(n, planes, per).int()
    start = torch.randint(1000, max_len - w, (n,), generator=g)
    d0 = torch.randint(0, planes, (n,), generator=g)
    seq_tables, seq_len, cu, row_len, src_row = [], [], [0], [], []
    q_rows = torch.randn(n * w, hq, d, generator=g).bfloat16()
    new_k = (torch.randn(n * w, hkv, d, generator=g) * 4).bfloat16()
    new_v = (torch.randn(n * w, hkv, d, generator=g) * 4).bfloat16()
    for i in range(n):
        for pl in range(planes):
            js = [j for j in range(w) if (int(d0[i]) + j) % planes == pl]
            if not js:
                continue
            seq_tables.append(tables[i, pl])
            seq_len.append(int(start[i]) + max(js) + 1)
            for j in js:
                row_len.append(int(start[i]) + j + 1)
                src_row.append(i * w + j)
            cu.append(cu[-1] + len(js))
    seq_tables = torch.stack(seq_tables)
    seq_len, cu = torch.tensor(seq_len, dtype=torch.int32), torch.tensor(cu, dtype=torch.int32)
    row_len, src_row = torch.tensor(row_len, dtype=torch.int32), torch.tensor(src_row)
    q, kn, vn = q_rows[src_row], new_k[src_row], new_v[src_row]
    sk, sv = torch.tensor(0.04, device=dev), torch.tensor(0.05, device=dev)
    seq_of_row = torch.repeat_interleave(torch.arange(len(seq_len)), cu[1:] - cu[:-1])
    pos = row_len.long() - 1
    blocks, offs = seq_tables.long()[seq_of_row, pos // bs], pos % bs
    max_q = int((cu[1:] - cu[:-1]).max())
    args = lambda kp, vp: (q.to(dev), kn.to(dev), vn.to(dev), kp, vp, seq_tables.to(dev),
                           seq_len.to(dev), cu.to(dev), max_q)
    # separate: K with the key scale, V with the value scale (store_fp8 takes one fixed
    # scale for both, so each pool is written by its own call), then prefill
    ka, va = kc.to(dev), vc.to(dev)
    scratch_k, scratch_v = ka.clone(), va.clone()
    sp = torch.zeros(pool, bs, hkv, device=dev)
    pkg.store_fp8(kn.to(dev), kn.to(dev), ka, scratch_v, sp, sp.clone(), blocks.to(dev),
                  offs.to(dev), 448.0, fixed_scale=0.04)
    pkg.store_fp8(vn.to(dev), vn.to(dev), scratch_k, va, sp.clone(), sp.clone(), blocks.to(dev),
                  offs.to(dev), 448.0, fixed_scale=0.05)
    want = kernel.prefill(q.to(dev), ka, va, seq_tables.to(dev), seq_len.to(dev), cu.to(dev),
                          max_q, sk, sv, row_lengths=row_len.to(dev))
    kb, vb = kc.to(dev), vc.to(dev)
    got = kernel.prefill_store(*args(kb, vb), sk, sv, row_lengths=row_len.to(dev))
    assert torch.equal(kb.view(torch.uint8), ka.view(torch.uint8))
    assert torch.equal(vb.view(torch.uint8), va.view(torch.uint8))
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # replayed from a graph: every replay gives the eager result
    kg, vg = kc.to(dev), vc.to(dev)
    a = args(kg, vg)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        kernel.prefill_store(*a, sk, sv, row_lengths=row_len.to(dev))
        rl = row_len.to(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = kernel.prefill_store(*a, sk, sv, row_lengths=rl)
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
        assert torch.equal(kg.view(torch.uint8), ka.view(torch.uint8))


def test_prefill_store_row_lengths_16bit_equals_store_then_prefill(kernel, pkg, dev):
    """Explicit row lengths on a 16-bit pool: rows stored at row_lengths - 1, in any
    order, then the row-lengths prefill, bit for bit (the one-launch form)."""
    _say("prefill_store row lengths bf16")
    g = torch.Generator().manual_seed(56)
    bs, hq, hkv, d = 16, 8, 2, 128
    lengths = [900, 1600]
    pages = sum(-(-x // bs) for x in lengths) + 3
    kpool, vpool, tables, q, k_new, v_new, cu = _window_store_case(
        g, torch.bfloat16, d, hq, hkv, bs, lengths, [3, 4], pages, layers=1, layer=0)
    row_len = torch.tensor([900, 896, 898, 1600, 1597, 1599, 1590], dtype=torch.int32)
    ctx = torch.tensor(lengths, dtype=torch.int32)
    seq = torch.tensor([0, 0, 0, 1, 1, 1, 1])
    pos = row_len.long() - 1
    ka, va = kpool.to(dev), vpool.to(dev)
    pkg.store_kv(ka[:, 0], va[:, 0], k_new.to(dev), v_new.to(dev),
                 tables.long()[seq, pos // bs].to(dev), (pos % bs).to(dev))
    want = kernel.prefill(q.to(dev), ka[:, 0], va[:, 0], tables.to(dev), ctx.to(dev), cu.to(dev),
                          4, row_lengths=row_len.to(dev))
    kb, vb = kpool.to(dev), vpool.to(dev)
    got = kernel.prefill_store(q.to(dev), k_new.to(dev), v_new.to(dev), kb[:, 0], vb[:, 0],
                               tables.to(dev), ctx.to(dev), cu.to(dev), 4,
                               row_lengths=row_len.to(dev))
    assert torch.equal(kb.view(torch.int16), ka.view(torch.int16))
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


# ------------------------------------------------------------ compensated P V

@pytest.mark.parametrize("d", [256, 128])
def test_compensated_p_keeps_small_value_residual(pkg, dev, d):
    """Reference known answer (tests/test_dory_gpu.py:501-517): two keys whose weighted
    values nearly cancel; rounding the weights to bf16 before P V moves the result, the
    compensated product keeps it (atol 5e-6 against the float64 closed form)."""
    _say("compensated KAT", d)
    q = torch.zeros((1, 1, d), dtype=torch.bfloat16)
    kv = torch.zeros((1, 16, 1, d), dtype=torch.bfloat16)
    k, v = kv.clone(), kv.clone()
    # the score of key 1 is -0.5 (D = 256) or as close as a bf16 q allows (D = 128)
    q0 = 16.0 if d == 256 else 11.3125
    q[0, 0, 0], k[0, 1, 0, 0] = q0, -0.5
    v[0, 0, 0, 0], v[0, 1, 0, 0] = -0.60546875, 1
    s1 = q0 * -0.5 / math.sqrt(d)
    w0, w1 = 1 / (1 + math.exp(s1)), math.exp(s1) / (1 + math.exp(s1))
    expected = w0 * -0.60546875 + w1 * 1.0
    assert expected > 0.0006
    table = torch.tensor([[0]], dtype=torch.int32)
    length = torch.tensor([2], dtype=torch.int32)
    cu = torch.tensor([0, 1], dtype=torch.int32)
    comp = pkg.MI355XPagedAttention(compensate=True)
    args = (q.to(dev), k.to(dev), v.to(dev), table.to(dev), length.to(dev))
    got = comp.prefill(*args, cu.to(dev), 1)
    assert abs(float(got[0, 0, 0]) - expected) <= 5e-6
    assert torch.equal(comp(*args), got)  # per-row == packed
    plain = pkg.MI355XPagedAttention()(*args)
    assert abs(float(plain[0, 0, 0]) - expected) > 5e-6  # the uncompensated cast loses it


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_compensated_packed_matches_per_row_and_is_closer(pkg, dev, dtype):
    """Compensated verify windows: packed == per-row bit for bit and batch invariant;
    against the float64 closed form the error is no larger than the uncompensated one's
    and within the output rounding (bf16 2^-8, fp16 2^-11 of the value, plus 1e-4)."""
    _say("compensated window", dtype)
    g = torch.Generator().manual_seed(31)
    bs, hq, hkv, d = 16, 16, 4, 128
    seqs = [(700, 5), (1500, 5), (33, 5), (4097, 9)]
    pages = sum(-(-n // bs) for n, _ in seqs) + 2
    _, _, k, v = make_pool(pages, 1, bs, hkv, d, dtype, g)
    tables = random_tables([n for n, _ in seqs], bs, pages, g)
    total = sum(c for _, c in seqs)
    q = torch.randn(total, hq, d, generator=g).to(dtype)
    lengths = torch.tensor([n for n, _ in seqs], dtype=torch.int32)
    cu = torch.tensor([0] + list(torch.tensor([c for _, c in seqs]).cumsum(0)), dtype=torch.int32)
    comp = pkg.MI355XPagedAttention(compensate=True)
    plain = pkg.MI355XPagedAttention()
    a = (q.to(dev), k.to(dev), v.to(dev), tables.to(dev), lengths.to(dev), cu.to(dev), 9)
    got = comp.prefill(*a).cpu()
    got_plain = plain.prefill(*a).cpu()
    # per-row form: each row its own table and length
    seq = torch.repeat_interleave(torch.arange(len(seqs)), torch.tensor([c for _, c in seqs]))
    i = torch.arange(total) - cu.long()[seq]
    row_len = lengths.long()[seq] - torch.tensor([c for _, c in seqs])[seq] + i + 1
    rows = comp(q.to(dev), k.to(dev), v.to(dev), tables[seq].to(dev), row_len.int().to(dev)).cpu()
    assert torch.equal(rows.view(torch.int16), got.view(torch.int16))
    one = comp.prefill(q[:5].to(dev), k.to(dev), v.to(dev), tables[:1].to(dev), lengths[:1].to(dev),
                       cu[:2].to(dev), 5).cpu()
    assert torch.equal(one.view(torch.int16), got[:5].view(torch.int16))
    err_c = err_p = 0.0
    rel = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    for s, (n, c) in enumerate(seqs):
        pages_s = tables[s, : -(-n // bs)].long()
        ks = k[pages_s].reshape(-1, hkv, d)[:n].double()
        vs = v[pages_s].reshape(-1, hkv, d)[:n].double()
        kk = ks.repeat_interleave(hq // hkv, 1).transpose(0, 1)
        vv = vs.repeat_interleave(hq // hkv, 1).transpose(0, 1)
        qq = q[cu[s]:cu[s + 1]].double().transpose(0, 1)
        sc = qq @ kk.transpose(1, 2) / math.sqrt(d)
        pos = torch.arange(n - c, n).view(-1, 1)
        sc = sc.masked_fill(torch.arange(n).view(1, -1) > pos, float("-inf"))
        want = (torch.softmax(sc, -1) @ vv).transpose(0, 1)
        gc, gp = got[cu[s]:cu[s + 1]].double(), got_plain[cu[s]:cu[s + 1]].double()
        assert ((gc - want).abs() <= rel * want.abs() + 1e-4).all()
        err_c = max(err_c, float((gc - want).abs().max()))
        err_p = max(err_p, float((gp - want).abs().max()))
    assert err_c <= err_p


def test_packed_window_shape_selects_compensation(pkg, dev):
    # reference: vllm_rlt/attention/backend.py:146-161 (a packed window shape opts in)
    shape = type("PackedWindowShape", (), {})()
    b = pkg.create_backend("auto", dev, torch.bfloat16, 128, 16, packed_window_shape=shape)
    assert b.info["compensated_p"] and b.kernel.compensate
    assert not pkg.create_backend("auto", dev, torch.bfloat16, 128, 16).kernel.compensate
    assert not pkg.create_backend("auto", dev, torch.float16, 128, 16,
                                  packed_window_shape=shape).kernel.compensate
