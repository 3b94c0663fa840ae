"""gfx950 acceptance sampler: reference known answers, and bit-exact parity with
the torch-CPU oracle on seeded inputs shaped like BASELINE.json configs 1 and 3-5."""

import sys
import types

import numpy as np
import pytest
import torch

from oracle import sampling as osamp
from tests import kat_sampling as kats

pytestmark = pytest.mark.gpu


def _say(*args):
    print("[case]", *args, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def impl(pkg, dev):
    return types.SimpleNamespace(categorical=pkg.categorical, speculative_accept=pkg.speculative_accept)


@pytest.mark.parametrize("kat", kats.ALL_KATS, ids=lambda f: f.__name__)
def test_gpu_known_answers(impl, dev, kat):
    _say(kat.__name__)
    kat(impl, dev)


@pytest.mark.parametrize("V", [1, 3, 5, 8, 9, 31, 32, 33, 100, 511, 512, 513, 4096, 8191, 8192,
                               8193, 12345, 49152, 65536, 70001, 262144 + 77])
def test_row_mass_is_torch_cpu_sum_bitwise(pkg, dev, V):
    _say("row_mass", V)
    g = torch.Generator().manual_seed(V)
    x = torch.rand(5, V, generator=g)
    x[0] = x[0] ** 8
    x[1] = x[1] * 1e-38
    x[2] = torch.randn(V, generator=g) * 1e6
    x[3] = torch.softmax(torch.randn(V, generator=g) * 3, -1)
    want = x.sum(-1, dtype=torch.float32)
    got = pkg.sampling.row_mass(x.to(dev)).cpu()
    assert np.array_equal(want.numpy().view(np.int32), got.numpy().view(np.int32))


def _verify_inputs(n, w1, vocab, g, temperature=1.0, top_p=1.0, noise=1.0, draft_std=3.0):
    """BASELINE config shape: draft logits ~N(0, draft_std^2), target = draft + N(0, noise^2)."""
    dl = torch.randn(n, w1 + 1, vocab, generator=g) * draft_std
    tl = dl + torch.randn(n, w1 + 1, vocab, generator=g) * noise
    t = torch.full((n * w1,), temperature)
    k = torch.full((n * w1,), -1, dtype=torch.int64)
    pp = torch.full((n * w1,), top_p)
    q = osamp.batched_probabilities(dl[:, :w1].reshape(-1, vocab), t, k, pp, max_top_k=0,
                                    apply_top_p=top_p < 1).view(n, w1, vocab)
    t2 = torch.full((n * (w1 + 1),), temperature)
    p = osamp.batched_probabilities(tl.reshape(-1, vocab), t2, torch.full_like(t2, -1).long(),
                                    torch.full_like(t2, top_p), max_top_k=0,
                                    apply_top_p=top_p < 1).view(n, w1 + 1, vocab)
    u = osamp.request_uniforms(torch.randint(0, 2**31, (n,), generator=g).tolist(), w1)
    drafts_tok = torch.stack([osamp.categorical(q[:, j], u[:, j])[0] for j in range(w1)], 1)
    return q, p, u, drafts_tok


def _check_accept(pkg, dev, q, p, u, draft_tokens, drafts):
    w1 = draft_tokens.shape[1]
    ua, uf = u[:, w1:2 * w1].contiguous(), u[:, 2 * w1].contiguous()
    want = osamp.speculative_accept(draft_tokens, drafts, q, p, ua, uf)
    got = pkg.speculative_accept(draft_tokens.to(dev), drafts.to(dev), q.to(dev), p.to(dev),
                                 ua.to(dev), uf.to(dev))
    for a, b, name in zip(got, want, want._fields):
        assert torch.equal(a.cpu(), b), name
    return want


@pytest.mark.parametrize("name,n,vocab,temperature,top_p", [
    ("config1", 8, 49152, 1.0, 1.0),
    ("config3", 32, 49152, 0.7, 0.9),
    ("config4", 16, 65536, 1.0, 1.0),
    ("config5", 64, 65536, 1.0, 1.0),
])
def test_accept_bit_exact_on_baseline_configs(pkg, dev, name, n, vocab, temperature, top_p):
    _say("accept", name)
    g = torch.Generator().manual_seed(hash(name) % 1000)
    w1 = 4
    q, p, u, dt = _verify_inputs(n, w1, vocab, g, temperature, top_p)
    drafts = torch.full((n,), w1, dtype=torch.int64)
    want = _check_accept(pkg, dev, q, p, u, dt, drafts)
    assert not want.error.any()


def test_accept_ragged_drafts_and_poisoned_padding(pkg, dev):
    _say("accept ragged")
    g = torch.Generator().manual_seed(77)
    n, w1, vocab = 40, 4, 3000
    q, p, u, dt = _verify_inputs(n, w1, vocab, g, noise=0.3)
    drafts = torch.randint(0, w1 + 1, (n,), generator=g)
    for i in range(n):
        d = int(drafts[i])
        q[i, d:] = float("nan")
        p[i, d + 1:] = float("nan")
    drafts[3] = 7  # out of range count: flagged, not honoured
    drafts[4] = -1
    dt[5, 0] = vocab + 3  # out-of-range token
    _check_accept(pkg, dev, q, p, u, dt, drafts)


@pytest.mark.parametrize("w1,vocab", [(1, 4099), (8, 12289), (32, 4097), (32, 8190)])
def test_accept_draft_widths_and_unaligned_vocab(pkg, dev, w1, vocab):
    """Draft widths 1 to 32 (the kernels' limit) with vocabularies that are not a multiple of
    4, so the weights take the scalar load path; low target noise makes long accepted runs, and
    ragged draft counts put the stop row at every depth."""
    _say("accept widths", w1, vocab)
    g = torch.Generator().manual_seed(w1 * 100003 + vocab)
    n = 12
    q, p, u, dt = _verify_inputs(n, w1, vocab, g, noise=0.02)
    drafts = torch.randint(0, w1 + 1, (n,), generator=g)
    drafts[0] = w1
    drafts[1] = 0
    want = _check_accept(pkg, dev, q, p, u, dt, drafts)
    assert not want.error.any()


def test_accept_high_acceptance_and_unnormalized_weights(pkg, dev):
    _say("accept unnormalized")
    g = torch.Generator().manual_seed(78)
    n, w1, vocab = 24, 4, 49152
    q, p, u, dt = _verify_inputs(n, w1, vocab, g, noise=0.05)
    q = q * torch.rand(n, w1, 1, generator=g) * 7  # raw weights: normalized inside
    p = p * torch.rand(n, w1 + 1, 1, generator=g) * 3
    _check_accept(pkg, dev, q, p, u, dt, torch.full((n,), w1, dtype=torch.int64))


@pytest.mark.parametrize("vocab", [1, 2, 7, 2047, 2048, 2049, 49152, 65536])
def test_categorical_bit_exact_random(pkg, dev, vocab):
    _say("categorical", vocab)
    g = torch.Generator().manual_seed(vocab)
    m = 64
    w = torch.rand(m, vocab, generator=g) ** 6
    w[w < 0.05] = 0
    w[1] = 0
    w[2, vocab // 2] = float("nan")
    u = torch.rand(m, generator=g)
    u[3], u[4], u[5] = 0.0, kats.BELOW_ONE, 1.0
    want = osamp.categorical(w, u)
    got = pkg.categorical(w.to(dev), u.to(dev))
    assert torch.equal(got[0].cpu(), want[0]) and torch.equal(got[1].cpu(), want[1])


def test_categorical_boundary_thresholds_take_the_exact_path(pkg, dev):
    # Thresholds placed exactly on cumulative boundaries (dyadic weights, exact
    # sums): the fast path cannot certify them, so the sequential replay decides.
    _say("categorical boundaries")
    vocab = 5000
    w = torch.zeros(vocab)
    w[::7] = 0.25
    w[3::11] = 0.5
    m = 256
    c = w.double().cumsum(0)
    mass = c[-1].item()
    picks = torch.linspace(0, vocab - 1, m).long()
    u = (c[picks] / mass).float()
    u = torch.where(u >= 1, torch.tensor(kats.BELOW_ONE), u)
    ww = w.expand(m, -1).contiguous()
    want = osamp.categorical(ww, u)
    got = pkg.categorical(ww.to(dev), u.to(dev))
    assert torch.equal(got[0].cpu(), want[0]) and torch.equal(got[1].cpu(), want[1])


def test_inputs_are_not_modified(pkg, dev):
    g = torch.Generator().manual_seed(9)
    q, p, u, dt = _verify_inputs(4, 3, 777, g)
    args = [dt.to(dev), torch.full((4,), 3).to(dev), q.to(dev), p.to(dev),
            u[:, 3:6].contiguous().to(dev), u[:, 6].contiguous().to(dev)]
    before = [a.clone() for a in args]
    pkg.speculative_accept(*args)
    torch.cuda.synchronize()
    for a, b in zip(args, before):
        assert torch.equal(a, b)


# ------------------------------------------------------------ random-round merge

def _merge_on_gpu(pkg, dev, args, res):
    target, accepted, next_tokens, starts, inputs, req, vrow, vrank, voff = args
    gres = pkg.AcceptResult(*(x.to(dev) for x in res))
    out = pkg.merge_random_round(target.to(dev), accepted.to(dev), next_tokens.to(dev),
                                 starts.to(dev), inputs.to(dev), gres, req.to(dev), vrow.to(dev),
                                 vrank.to(dev), voff.to(dev))
    return [x.cpu() for x in out]


def test_merge_random_round_known_answer(pkg, dev):
    # reference: tests/test_async_speculative_sampling_plan.py:127-161
    _say("merge KAT")
    res = osamp.AcceptResult(tokens=torch.tensor([[77, 66, 55], [9, 0, 0]]),
                             accepted=torch.tensor([2, 0]), final=torch.tensor([55, 0]),
                             error=torch.tensor([False, True]))
    args = (torch.tensor([10, 11, 12, 20, 21, 30, 31]), torch.tensor([0, 1, 0]),
            torch.tensor([10, 21, 30]), torch.tensor([5, 8, 12]), torch.tensor([1, 2, 3]),
            torch.tensor([0, 2]), torch.tensor([0, 1, 2, 5, 6]), torch.tensor([0, 0, 0, 1, 1]),
            torch.tensor([0, 1, 2, 0, 1]))
    rows, acc, nxt, pos, values, err = _merge_on_gpu(pkg, dev, args, res)
    assert rows.tolist() == [77, 66, 55, 20, 21, 9, 0]
    assert acc.tolist() == [2, 1, 0] and nxt.tolist() == [55, 21, 0]
    assert pos.tolist() == [8, 10, 13]
    assert values.tolist() == [[55, 8], [21, 10], [3, 12]]
    assert err.tolist() == [0, 0, 1] and err.dtype == torch.int64


@pytest.mark.parametrize("n,seed", [(1, 0), (7, 1), (300, 2), (2500, 3)])
def test_merge_random_round_matches_oracle(pkg, dev, n, seed):
    _say("merge", n, seed)
    g = torch.Generator().manual_seed(seed)
    k = 4
    temps = (torch.rand(n, generator=g) < 0.6).float() * 0.7
    counts = torch.randint(1, k + 2, (n,), generator=g).tolist()
    plan = osamp.plan_random_rows(temps.tolist(), counts, k)
    total = sum(counts)
    target = torch.randint(0, 50000, (total,), generator=g)
    accepted = torch.randint(0, k + 1, (n,), generator=g)
    next_tokens = torch.randint(0, 50000, (n,), generator=g)
    starts = torch.randint(0, 10000, (n,), generator=g)
    inputs = torch.randint(0, 50000, (n,), generator=g)
    if plan is None:
        req = vrow = vrank = voff = torch.zeros(0, dtype=torch.int64)
    else:
        req, vrow, vrank, voff = (torch.as_tensor(x, dtype=torch.int64) for x in plan)
    r = req.shape[0]
    res = osamp.AcceptResult(tokens=torch.randint(0, 50000, (r, k + 1), generator=g),
                             accepted=torch.randint(0, k + 1, (r,), generator=g),
                             final=torch.randint(0, 50000, (r,), generator=g),
                             error=torch.rand(r, generator=g) < 0.2)
    args = (target, accepted, next_tokens, starts, inputs, req, vrow, vrank, voff)
    got = _merge_on_gpu(pkg, dev, args, res)
    want = osamp.merge_random_round(target, accepted, next_tokens, starts, inputs, res, req, vrow,
                                    vrank, voff)
    for a, b in zip(got, want):
        assert torch.equal(a, b.reshape(a.shape).to(a.dtype))


@pytest.mark.parametrize("corrupt", ["row", "rank", "offset", "request"])
def test_merge_random_round_corrupt_plan_fails_the_round(pkg, dev, corrupt):
    """An index outside its range: the reference's indexing raises; the device merge
    skips it and reports every request failed, each keeping its slot values."""
    _say("merge corrupt", corrupt)
    res = osamp.AcceptResult(tokens=torch.tensor([[77, 66, 55], [9, 0, 0]]),
                             accepted=torch.tensor([2, 0]), final=torch.tensor([55, 0]),
                             error=torch.tensor([False, False]))
    vrow, vrank = torch.tensor([0, 1, 2, 5, 6]), torch.tensor([0, 0, 0, 1, 1])
    voff, req = torch.tensor([0, 1, 2, 0, 1]), torch.tensor([0, 2])
    if corrupt == "row":
        vrow[3] = 7
    elif corrupt == "rank":
        vrank[4] = 2
    elif corrupt == "offset":
        voff[2] = 3
    else:
        req[1] = 3
    args = (torch.tensor([10, 11, 12, 20, 21, 30, 31]), torch.tensor([0, 1, 0]),
            torch.tensor([10, 21, 30]), torch.tensor([5, 8, 12]), torch.tensor([1, 2, 3]),
            req, vrow, vrank, voff)
    with pytest.raises(IndexError):
        osamp.merge_random_round(*args[:5], res, *args[5:])
    rows, acc, nxt, pos, values, err = _merge_on_gpu(pkg, dev, args, res)
    assert err.tolist() == [1, 1, 1]
    assert values.tolist() == [[1, 5], [2, 8], [3, 12]]


# ------------------------------------- against the reference formula on the device

def _margins(q, p, u, dt, w1):
    """Per request: the smallest relative margin of any decision the reference takes
    (each accept test u*qx < px up to the stop point, and the final inverse-CDF
    threshold against the cumulative values around the drawn index), in torch-CPU
    arithmetic."""
    ua, uf = u[:, w1:2 * w1], u[:, 2 * w1]
    res = osamp.speculative_accept(dt, torch.full((dt.shape[0],), w1), q, p, ua, uf)
    pm, qm = p.sum(-1, dtype=torch.float32), q.sum(-1, dtype=torch.float32)
    out = []
    for i in range(dt.shape[0]):
        s = int(res.accepted[i])
        m = float("inf")
        for j in range(min(s + 1, w1)):
            x = int(dt[i, j])
            px, qx = float(p[i, j, x] / pm[i, j]), float(q[i, j, x] / qm[i, j])
            m = min(m, abs(float(ua[i, j]) * qx - px) / max(px, 1e-30), abs(px - qx) / max(px, 1e-30))
        pr = p[i, s].double() / float(pm[i, s])
        w = pr if s == w1 else (pr - q[i, s].double() / float(qm[i, s])).clamp_min(0)
        c = w.cumsum(0)
        t = float(uf[i]) * float(c[-1])
        k = int(res.final[i])
        lo = float(c[k - 1]) if k > 0 else 0.0
        m = min(m, abs(t - lo) / float(c[-1]), abs(float(c[k]) - t) / float(c[-1]))
        out.append(m)
    return out


@pytest.mark.parametrize("name,n,vocab,temperature,top_p", [
    ("config1", 8, 49152, 1.0, 1.0),
    ("config3", 32, 49152, 0.7, 0.9),
    ("config5", 256, 65536, 1.0, 1.0),
])
def test_accept_against_reference_formula_run_on_the_gpu(pkg, dev, name, n, vocab, temperature,
                                                         top_p):
    """The reference's own async path runs speculative_accept on device tensors
    (vllm_rlt/worker/async_speculative.py:727-734), so its row sums and float64 cumsum
    follow torch-ROCm's reduction orders, not torch-CPU's that this kernel reproduces.
    Every request where the two disagree must hinge on a decision whose margin is
    within float32 rounding of the masses (relative 1e-5); on these seeds they agree."""
    _say("accept vs device reference", name)
    g = torch.Generator().manual_seed(1000 + n)
    w1 = 4
    q, p, u, dt = _verify_inputs(n, w1, vocab, g, temperature, top_p)
    drafts = torch.full((n,), w1, dtype=torch.int64)
    ua, uf = u[:, w1:2 * w1].contiguous(), u[:, 2 * w1].contiguous()
    args = [a.to(dev) for a in (dt, drafts, q, p, ua, uf)]
    ours = pkg.speculative_accept(*args)
    dev_ref = osamp.speculative_accept(*args)
    cpu_ref = osamp.speculative_accept(dt, drafts, q, p, ua, uf)
    assert torch.equal(ours.tokens.cpu(), cpu_ref.tokens)
    differ = [i for i in range(n)
              if not (torch.equal(ours.tokens[i].cpu(), dev_ref.tokens[i].cpu())
                      and int(ours.accepted[i]) == int(dev_ref.accepted[i]))]
    if differ:
        margins = _margins(q, p, u, dt, w1)
        assert all(margins[i] <= 1e-5 for i in differ), [(i, margins[i]) for i in differ]
    # the masses themselves: torch-ROCm's fp32 row sums are within a few ulps of ours
    gm = p.to(dev).sum(-1, dtype=torch.float32).cpu()
    cm = p.sum(-1, dtype=torch.float32)
    assert ((gm - cm).abs() <= 8 * torch.finfo(torch.float32).eps * cm.abs()).all()
    print(f"[case] {name}: {len(differ)} of {n} requests differ from the device reference",
          flush=True)


def test_order_fixture_sums_are_the_kernels(pkg, dev):
    """The constants the import-time guard compares the host's torch with are the
    kernels' own sums of the fixture rows."""
    from vllm_rlt_amd import sampling

    for vocab, bits in sampling.ORDER_FIXTURE_SUMS.items():
        x = torch.from_numpy(sampling.order_fixture(vocab)).view(1, vocab).repeat(3, 1)
        got = pkg.sampling.row_mass(x.to(dev)).cpu()
        assert all((int(v) & 0xFFFFFFFF) == bits for v in got.view(torch.int32)), vocab
