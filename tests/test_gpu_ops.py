"""torch.ops.rlt_mi355x operators on the GPU: same results as the package API, and
torch.library.opcheck's schema and fake-tensor checks."""

import pytest
import torch

from tests.attn_cases import make_pool, random_tables

pytestmark = pytest.mark.gpu
CHECKS = ("test_schema", "test_faketensor")


def test_attention_and_sampling_ops_match_the_api(pkg, dev):
    g = torch.Generator().manual_seed(1)
    _, _, k, v = make_pool(40, 1, 16, 4, 128, torch.bfloat16, g)
    lengths = torch.tensor([100, 37, 300], dtype=torch.int32)
    tables = random_tables(lengths.tolist(), 16, 40, g)
    q = torch.randn(15, 16, 128, generator=g).bfloat16()
    cu = torch.tensor([0, 5, 10, 15], dtype=torch.int32)
    args = (q.to(dev), k.to(dev), v.to(dev), tables.to(dev), lengths.to(dev), None, None,
            cu.to(dev), 5, 0)
    got = torch.ops.rlt_mi355x.paged_attention(*args)
    want = pkg.MI355XPagedAttention().prefill(*args[:5], cu.to(dev), 5)
    assert torch.equal(got, want)
    torch.library.opcheck(torch.ops.rlt_mi355x.paged_attention, args, test_utils=CHECKS)

    # the window's K/V stored by the attention launch: the pool afterwards and the output
    # equal the separate store + attention (the pool is rewritten with the same rows)
    kn = torch.randn(15, 4, 128, generator=g).bfloat16().to(dev)
    vn = torch.randn(15, 4, 128, generator=g).bfloat16().to(dev)
    kd, vd = k.to(dev), v.to(dev)
    sa = (q.to(dev), kn, vn, kd, vd, tables.to(dev), lengths.to(dev), cu.to(dev), 5)
    got = torch.ops.rlt_mi355x.paged_attention_store(*sa)
    ks, vs = k.to(dev), v.to(dev)
    seq = torch.arange(3).repeat_interleave(5)
    pos = lengths.long()[seq] - 5 + torch.arange(15) % 5
    pkg.store_kv(ks, vs, kn, vn, tables.long()[seq, pos // 16].to(dev), (pos % 16).to(dev))
    want = pkg.MI355XPagedAttention().prefill(q.to(dev), ks, vs, tables.to(dev), lengths.to(dev),
                                              cu.to(dev), 5)
    assert torch.equal(got, want) and torch.equal(kd, ks) and torch.equal(vd, vs)
    torch.library.opcheck(torch.ops.rlt_mi355x.paged_attention_store, sa, test_utils=CHECKS)
    # an FP8 pool is refused before anything is stored (it needs scales)
    k8, v8 = kd.to(torch.float8_e4m3fn), vd.to(torch.float8_e4m3fn)
    k8_before = k8.view(torch.uint8).clone()
    with pytest.raises(ValueError, match="FP8"):
        torch.ops.rlt_mi355x.paged_attention_store(q.to(dev), kn.to(torch.float8_e4m3fn),
                                                   vn.to(torch.float8_e4m3fn), k8, v8,
                                                   tables.to(dev), lengths.to(dev), cu.to(dev), 5)
    assert torch.equal(k8.view(torch.uint8), k8_before)

    logits = torch.randn(6, 3000, generator=g).to(dev)
    t, tk = torch.full((6,), 0.8, device=dev), torch.full((6,), -1, dtype=torch.int64, device=dev)
    tp = torch.full((6,), 0.9, device=dev)
    pa = (logits, t, tk, tp, 0, True)
    probs = torch.ops.rlt_mi355x.spec_probs(*pa)
    assert torch.equal(probs, pkg.batched_probabilities(logits, t, tk, tp, max_top_k=0,
                                                        apply_top_p=True))
    torch.library.opcheck(torch.ops.rlt_mi355x.spec_probs, pa, test_utils=CHECKS)

    u = torch.rand(6, generator=g).to(dev)
    idx, valid = torch.ops.rlt_mi355x.categorical(probs, u)
    want_idx, want_valid = pkg.categorical(probs, u)
    assert torch.equal(idx, want_idx) and torch.equal(valid, want_valid)

    n, w1 = 2, 2
    pq = probs[: n * (w1 + 1)].view(n, w1 + 1, -1).contiguous()
    qq = probs[: n * w1].view(n, w1, -1).contiguous()
    dt = torch.stack([pkg.categorical(qq[:, j].contiguous(), u[:n])[0] for j in range(w1)], 1)
    drafts = torch.full((n,), w1, dtype=torch.int64, device=dev)
    ua, uf = torch.rand(n, w1, generator=g).to(dev), torch.rand(n, generator=g).to(dev)
    got = torch.ops.rlt_mi355x.spec_accept(dt, drafts, qq, pq, ua, uf)
    want = pkg.speculative_accept(dt, drafts, qq, pq, ua, uf)
    for a, b in zip(got, want):
        assert torch.equal(a, b)

    va = (logits[: n * (w1 + 1)].view(n, w1 + 1, -1), t[: n * (w1 + 1)], tk[: n * (w1 + 1)],
          tp[: n * (w1 + 1)], dt, drafts, qq, ua, uf, 0, True)
    got = torch.ops.rlt_mi355x.verify_accept(*va)
    want_t, want_p, want_r = pkg.verify_accept(*va[:9], max_top_k=0, apply_top_p=True)
    for a, b in zip(got, (want_t, want_p) + tuple(want_r)):
        assert torch.equal(a, b)
    torch.library.opcheck(torch.ops.rlt_mi355x.verify_accept, va, test_utils=CHECKS)


def test_kv_write_op_mutates_the_pool(pkg, dev):
    kc = torch.zeros(8, 16, 2, 64, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    k = torch.randn(3, 2, 64, device=dev).bfloat16()
    blocks = torch.tensor([1, 5, 7], device=dev)
    offsets = torch.tensor([0, 15, 3], device=dev)
    torch.ops.rlt_mi355x.store_kv(kc, vc, k, -k, blocks, offsets, None, None)
    assert torch.equal(kc[blocks, offsets], k) and torch.equal(vc[blocks, offsets], -k)


def test_merge_random_round_op(pkg, dev):
    # reference KAT: tests/test_async_speculative_sampling_plan.py:127-161
    t = lambda x, **kw: torch.tensor(x, device=dev, **kw)  # noqa: E731
    args = (t([10, 11, 12, 20, 21, 30, 31]), t([0, 1, 0]), t([10, 21, 30]), t([5, 8, 12]),
            t([1, 2, 3]), t([[77, 66, 55], [9, 0, 0]]), t([2, 0]), t([55, 0]),
            t([False, True]), t([0, 2]), t([0, 1, 2, 5, 6]), t([0, 0, 0, 1, 1]), t([0, 1, 2, 0, 1]))
    rows, acc, nxt, pos, values, err = torch.ops.rlt_mi355x.merge_random_round(*args)
    assert rows.tolist() == [77, 66, 55, 20, 21, 9, 0]
    assert acc.tolist() == [2, 1, 0] and nxt.tolist() == [55, 21, 0] and pos.tolist() == [8, 10, 13]
    assert values.tolist() == [[55, 8], [21, 10], [3, 12]] and err.tolist() == [0, 0, 1]
    torch.library.opcheck(torch.ops.rlt_mi355x.merge_random_round, args, test_utils=CHECKS)


def test_ops_raise_on_host_tensors_and_on_conversions_they_would_need(pkg, dev):
    """The C++ operators raise ValueError -- before any launch -- for a host tensor next
    to device tensors (its pointer would fault the GPU), and for a dtype or layout they
    do not read (no hidden copy); the package functions make the conversions the
    reference's own functions make and give the same result."""
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(4, 1000, generator=g).to(dev)
    t, tk = torch.full((4,), 0.8, device=dev), torch.full((4,), -1, dtype=torch.int64, device=dev)
    tp = torch.full((4,), 0.9, device=dev)
    with pytest.raises(ValueError, match="device"):
        torch.ops.rlt_mi355x.spec_probs(logits, t.cpu(), tk, tp, 0, True)
    with pytest.raises(ValueError, match="top_k"):
        torch.ops.rlt_mi355x.spec_probs(logits, t, tk.int(), tp, 0, True)
    want = torch.ops.rlt_mi355x.spec_probs(logits, t, tk, tp, 0, True)
    assert torch.equal(pkg.batched_probabilities(logits.double(), t.half(), tk.int(), tp,
                                                 max_top_k=0, apply_top_p=True),
                       torch.ops.rlt_mi355x.spec_probs(logits.double().float(),
                                                       t.half().float(), tk, tp, 0, True))
    u = torch.rand(4, generator=g).to(dev)
    with pytest.raises(ValueError, match="device"):
        torch.ops.rlt_mi355x.categorical(want, u.cpu())
    with pytest.raises(ValueError, match="weights"):
        torch.ops.rlt_mi355x.categorical(want.t().contiguous().t(), u)
    idx, _ = pkg.categorical(want.t().contiguous().t(), u)
    assert torch.equal(idx, torch.ops.rlt_mi355x.categorical(want, u)[0])

    _, _, k, v = make_pool(40, 1, 16, 4, 128, torch.bfloat16, g)
    lengths = torch.tensor([100, 37], dtype=torch.int32)
    tables = random_tables(lengths.tolist(), 16, 40, g)
    q = torch.randn(2, 8, 128, generator=g).bfloat16().to(dev)
    kd, vd = k.to(dev), v.to(dev)
    base = (q, kd, vd, tables.to(dev), lengths.to(dev), None, None, None, 1, 0)
    with pytest.raises(ValueError, match="device"):
        torch.ops.rlt_mi355x.paged_attention(*base[:3], tables, *base[4:])
    with pytest.raises(ValueError, match="block_tables"):
        torch.ops.rlt_mi355x.paged_attention(*base[:3], tables.long().to(dev), *base[4:])
    with pytest.raises(ValueError, match="context_lengths"):
        torch.ops.rlt_mi355x.paged_attention(*base[:4], lengths.long().to(dev), *base[5:])
    with pytest.raises(ValueError, match="head dimension"):
        qs = torch.randn(2, 128, 8, generator=g).bfloat16().to(dev).transpose(1, 2)
        torch.ops.rlt_mi355x.paged_attention(qs, *base[1:])

    kc = torch.zeros(8, 16, 2, 64, dtype=torch.bfloat16, device=dev)
    rows = torch.randn(2, 2, 64, device=dev).bfloat16()
    blocks, offsets = torch.tensor([1, 5], device=dev), torch.tensor([0, 3], device=dev)
    with pytest.raises(ValueError, match="device"):
        torch.ops.rlt_mi355x.store_kv(kc, kc.clone(), rows, rows, blocks.cpu(), offsets, None, None)
    with pytest.raises(ValueError, match="blocks"):
        torch.ops.rlt_mi355x.store_kv(kc, kc.clone(), rows, rows, blocks.int(), offsets, None, None)
    assert not kc.any()  # nothing was written by the refused calls
    pkg.store_kv(kc, kc.clone(), rows, rows, blocks.int(), offsets)
    assert torch.equal(kc[blocks, offsets], rows)
