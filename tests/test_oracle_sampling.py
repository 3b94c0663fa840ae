"""The CPU oracle against the reference's known answers and closed forms."""

import types

import pytest
import numpy as np
import torch

from oracle import sampling as osamp
from tests import kat_sampling as kats

ORACLE = types.SimpleNamespace(categorical=osamp.categorical,
                               speculative_accept=osamp.speculative_accept)


@pytest.mark.parametrize("kat", kats.ALL_KATS, ids=lambda f: f.__name__)
def test_oracle_known_answers(kat):
    kat(ORACLE, torch.device("cpu"))


def test_ragged_monte_carlo_matches_target():
    # reference: tests/test_speculative_sampling.py:366-426 (NaN-poisoned padding)
    vocab, w1, reps = 6, 3, 20_000
    counts = [0, 1, 2, 3, 3]
    g = torch.Generator().manual_seed(7)

    def rand_weights(*shape):
        w = torch.rand(*shape, generator=g) + 0.05
        w[torch.rand(*shape, generator=g) < 0.2] = 0.0
        w[..., 0] += 0.5
        return w

    q = rand_weights(len(counts), w1, vocab)
    p = rand_weights(len(counts), w1 + 1, vocab)
    drafts = torch.zeros(len(counts), reps, w1, dtype=torch.int64)
    for i, d in enumerate(counts):
        for j in range(d):
            drafts[i, :, j] = torch.multinomial(q[i, j], reps, replacement=True, generator=g)
    q_in, p_in = q.clone(), p.clone()
    for i, d in enumerate(counts):
        q_in[i, d:] = float("nan")
        p_in[i, d + 1:] = float("nan")
    n = len(counts) * reps
    rep = lambda t: t.repeat_interleave(reps, dim=0)  # noqa: E731
    out = osamp.speculative_accept(drafts.reshape(n, w1), rep(torch.tensor(counts)), rep(q_in),
                                   rep(p_in), torch.rand(n, w1, generator=g), torch.rand(n, generator=g))
    assert not out.error.any()
    tokens = out.tokens.view(len(counts), reps, w1 + 1)
    accepted = out.accepted.view(len(counts), reps)
    pn = p / p.sum(-1, keepdim=True)
    qn = q / q.sum(-1, keepdim=True)
    for i, d in enumerate(counts):
        assert (accepted[i] <= d).all()
        freq = torch.bincount(tokens[i, :, 0], minlength=vocab).double() / reps
        se = (pn[i, 0].double() * (1 - pn[i, 0].double()) / reps).sqrt()
        assert ((freq - pn[i, 0].double()).abs() <= 5 * se + 1e-6).all()
        reach = 1.0
        for k in range(1, d + 1):
            reach *= torch.minimum(pn[i, k - 1], qn[i, k - 1]).sum().item()
            hit = (accepted[i] >= k).double().mean().item()
            assert abs(hit - reach) <= 5 * (reach * (1 - reach) / reps) ** 0.5 + 1e-6


def test_probability_filter_closed_forms():
    # reference: tests/test_speculative.py:474-490
    logits = torch.tensor([0.50, 0.25, 0.15, 0.10]).log()
    p = osamp.sampler_probabilities(logits, 1.0, -1, 0.8)
    torch.testing.assert_close(p, torch.tensor([0.50, 0.25, 0.15, 0]) / 0.9)
    p = osamp.sampler_probabilities(logits, 0.5, 2, 1.0)
    torch.testing.assert_close(p, torch.tensor([0.8, 0.2, 0, 0]))
    p = osamp.sampler_probabilities(torch.zeros(4), 1.0, 1, 1.0)
    assert int((p > 0).sum()) == 1


def test_batched_probabilities_match_row_form():
    # reference: tests/test_speculative_sampling.py:44-60
    vocab = 17
    g = torch.Generator().manual_seed(0)
    top_ks = [-1, 1, 3, vocab, vocab + 5]
    top_ps = [1.0, 0.9, 0.5]
    temps = [0.5, 0.8, 1.0, 1.5, 2.0]
    tk = [top_ks[i % 5] for i in range(30)]
    tp = [top_ps[(i // 5) % 3] for i in range(30)]
    tt = [temps[(i * 3) % 5] for i in range(30)]
    logits = torch.randn(30, vocab, generator=g) * 3
    got = osamp.batched_probabilities(
        logits, torch.tensor(tt), torch.tensor(tk), torch.tensor(tp),
        max_top_k=max(k for k in tk if 0 < k < vocab), apply_top_p=True)
    want = torch.stack([osamp.sampler_probabilities(logits[i], tt[i], tk[i], tp[i]) for i in range(30)])
    torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-5)
    # top_p == 1 and untruncated rows are the plain softmax
    torch.testing.assert_close(got[0], (logits[0] / tt[0]).softmax(-1), atol=1e-6, rtol=1e-5)


def test_greedy_accept_known_answers():
    # reference: tests/test_speculative.py:276-285
    for k in (0, 1, 2, 4, 8):
        cands = list(range(100, 100 + k))
        for rejected in range(k + 1):
            targets = cands[:rejected] + [7] + list(range(200, 200 + k - rejected))
            tokens, accepted = osamp.greedy_accept(cands, targets)
            assert accepted == rejected and tokens == cands[:rejected] + [7]


def test_greedy_batched_matches_host_form_by_brute_force():
    g = torch.Generator().manual_seed(5)
    n, w1, vocab = 64, 4, 5
    logits = torch.randn(n, w1 + 1, vocab, generator=g)
    targets = logits.argmax(-1)
    drafts_tok = torch.where(torch.rand(n, w1, generator=g) < 0.7, targets[:, :w1],
                             torch.randint(0, vocab, (n, w1), generator=g))
    drafts = torch.randint(0, w1 + 1, (n,), generator=g)
    t, acc, nxt = osamp.greedy_accept_batched(drafts_tok, drafts, logits)
    for i in range(n):
        d = int(drafts[i])
        toks, a = osamp.greedy_accept(drafts_tok[i, :d].tolist(), targets[i, :d + 1].tolist())
        assert a == acc[i].item() and toks[-1] == nxt[i].item()


def test_merge_random_round_known_answer():
    # reference: tests/test_async_speculative_sampling_plan.py:127-161
    res = osamp.AcceptResult(tokens=torch.tensor([[77, 66, 55], [9, 0, 0]]),
                             accepted=torch.tensor([2, 0]), final=torch.tensor([55, 0]),
                             error=torch.tensor([False, True]))
    rows, acc, nxt, pos, values, err = osamp.merge_random_round(
        torch.tensor([10, 11, 12, 20, 21, 30, 31]), torch.tensor([0, 1, 0]), torch.tensor([10, 21, 30]),
        torch.tensor([5, 8, 12]), torch.tensor([1, 2, 3]), res, torch.tensor([0, 2]),
        torch.tensor([0, 1, 2, 5, 6]), torch.tensor([0, 0, 0, 1, 1]), torch.tensor([0, 1, 2, 0, 1]))
    assert rows.tolist() == [77, 66, 55, 20, 21, 9, 0]
    assert acc.tolist() == [2, 1, 0] and nxt.tolist() == [55, 21, 0]
    assert pos.tolist() == [8, 10, 13]
    assert values.tolist() == [[55, 8], [21, 10], [3, 12]]
    assert err.tolist() == [0, 0, 1] and err.dtype == torch.int64


def test_uniform_protocol_one_block_per_round():
    # reference: tests/test_async_speculative_sampling_plan.py:366-382
    k = 4
    u = osamp.request_uniforms([1, 3], k)
    for row, seed in zip(u, (1, 3)):
        ref = torch.Generator().manual_seed(seed)
        assert torch.equal(row, torch.rand((2 * k + 1,), generator=ref))


def test_accept_shape_errors():
    with pytest.raises(ValueError):
        osamp.speculative_accept(torch.zeros(2, 3, dtype=torch.long), torch.zeros(3, dtype=torch.long),
                                 torch.zeros(2, 3, 4), torch.zeros(2, 4, 4), torch.zeros(2, 3), torch.zeros(2))
    with pytest.raises(ValueError):
        osamp.categorical(torch.zeros(3), torch.zeros(3))


# ------------------------------------------------ synchronous runner's rejection sampling

@pytest.mark.parametrize("p,q", [
    ([0.1, 0.6, 0.3], [0.7, 0.2, 0.1]),
    ([0.0, 1.0, 0.0], [1.0, 0.0, 0.0]),
    ([0.2, 0.3, 0.5], [0.2, 0.3, 0.5]),
])
def test_rejection_sample_recovers_target_distribution(p, q):
    # reference known answer: tests/test_speculative.py:455-471
    p, q = torch.tensor(p), torch.tensor(q)
    g = torch.Generator().manual_seed(431)
    counts = torch.zeros(3)
    for _ in range(12000):
        candidate = int(torch.multinomial(q, 1, generator=g))
        token, _ = osamp.rejection_sample(candidate, p, q, g)
        counts[token] += 1
    torch.testing.assert_close(counts / counts.sum(), p, atol=0.016, rtol=0)


def test_rejection_step_closed_form_and_errors():
    p = torch.tensor([0.1, 0.6, 0.3])
    q = torch.tensor([0.7, 0.2, 0.1])
    assert osamp.rejection_step(1, p, q, torch.tensor(0.99))[0]  # p >= q: always accepted
    ok, r = osamp.rejection_step(0, p, q, torch.tensor(0.5))  # 0.35 >= 0.1: rejected
    assert not ok
    p32, q32 = p.numpy(), q.numpy()
    diff = np.maximum(p32 - q32, np.float32(0))
    want = diff / ((diff[0] + diff[1]) + diff[2])
    assert np.array_equal(r.numpy(), want)
    with pytest.raises(ValueError):
        osamp.rejection_step(0, p, torch.tensor([0.0, 0.5, 0.5]), torch.tensor(0.1))
    with pytest.raises(RuntimeError):
        osamp.rejection_step(0, torch.tensor([0.1, float("nan"), 0.3]), q, torch.tensor(0.5))


def test_collect_stochastic_consumes_the_generator_like_the_loop():
    """One uniform per examined draft, then one multinomial draw: the generator of a
    request that accepts everything advances by K uniforms and the bonus draw."""
    p = torch.tensor([[[0.0, 1.0], [0.0, 1.0], [0.5, 0.5]]])
    q = torch.tensor([[[0.0, 1.0], [0.0, 1.0]]])
    g = torch.Generator().manual_seed(3)
    res = osamp.collect_stochastic([[1, 1]], p, q, [g])
    assert res[0][1] == 2 and res[0][0][:2] == [1, 1]
    h = torch.Generator().manual_seed(3)
    torch.rand((), generator=h), torch.rand((), generator=h)
    torch.multinomial(p[0, 2], 1, generator=h)
    assert torch.equal(g.get_state(), h.get_state())
