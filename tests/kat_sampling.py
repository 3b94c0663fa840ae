"""Known-answer tests of the acceptance sampler, shared by the oracle (CPU) and
the gfx950 implementation (GPU).

Transcribed from the reference's tests/test_speculative_sampling.py:149-576 (the
exact inputs and expected answers, re-expressed as data + checks).  Each check
takes ``impl`` = an object with ``categorical(w, u)`` and
``speculative_accept(...)`` and a torch ``device``.
"""

import torch

BELOW_ONE = torch.nextafter(torch.tensor(1.0), torch.tensor(0.0)).item()
NAN = float("nan")
E0, E1, E2, E3 = ([1.0 if i == j else 0.0 for i in range(4)] for j in range(4))
BAD = [NAN] * 4


def _cat(impl, rows, u, device):
    idx, valid = impl.categorical(torch.as_tensor(rows, dtype=torch.float32).to(device),
                                  torch.as_tensor(u, dtype=torch.float32).to(device))
    return idx.cpu(), valid.cpu()


def kat_categorical_midpoint_quadrature(impl, device):
    m = 4096
    w = torch.tensor([3.0, 0.0, 1.0, 4.0, 0.5, 0.0, 2.5])
    u = ((torch.arange(m, dtype=torch.float64) + 0.5) / m).float()
    idx, valid = _cat(impl, w.expand(m, -1).contiguous(), u, device)
    assert valid.all()
    freq = torch.bincount(idx, minlength=7).double() / m
    assert (freq - (w / w.sum()).double()).abs().max() <= 1 / m + 1e-9
    assert freq[w == 0].sum() == 0


def kat_categorical_trailing_zeros(impl, device):
    for weight in (1.0, 1 / 41):
        row = torch.tensor([weight] * 41 + [0.0, 0.0], dtype=torch.float32)
        mass32 = row.cumsum(-1)[-1].item()
        probes = [BELOW_ONE]
        for _ in range(3):
            probes.append(torch.nextafter(torch.tensor(probes[-1]), torch.tensor(0.0)).item())
        if mass32 < 1:
            probes.append(mass32)
        idx, valid = _cat(impl, row.expand(len(probes), -1).contiguous(), probes, device)
        assert valid.all()
        assert (idx < 41).all()
        assert idx[0] == 40


def kat_categorical_out_of_contract_uniform(impl, device):
    row = torch.tensor([1.0] * 41 + [0.0, 0.0])
    idx, valid = _cat(impl, row.expand(2, -1).contiguous(), [1.0, 1.5], device)
    assert valid.all() and idx.tolist() == [40, 40]


def kat_categorical_small_token_after_large_mass(impl, device):
    upper = torch.tensor(1 - 0.25e-6, dtype=torch.float32).item()
    idx, valid = _cat(impl, torch.tensor([[1.0, 1e-6]] * 3), [0.5, upper, 0.999998], device)
    assert valid.all() and idx.tolist() == [0, 1, 0]


def kat_categorical_fp64_cdf(impl, device):
    idx, _ = _cat(impl, torch.tensor([[1.0, 1e-5]] * 2), [0.9999899864196777, 0.99999499], device)
    assert idx.tolist() == [0, 1]


def kat_categorical_exact_boundaries(impl, device):
    idx, valid = _cat(impl, torch.tensor([[0.0, 1.0, 0.0, 3.0]] * 3), [0.0, 0.25, 0.5], device)
    assert valid.all() and idx.tolist() == [1, 3, 3]


def kat_categorical_plateau_tail(impl, device):
    idx, valid = _cat(impl, torch.tensor([[1.0, 1e-20]] * 4), [0.0, 0.5, 0.999, BELOW_ONE], device)
    assert valid.all() and (idx == 0).all()


def kat_categorical_invalid_rows(impl, device):
    inf = float("inf")
    w = [[0.0, 0.0, 0.0], [0.0, 1.0, 0.0], [1.0, NAN, 1.0], [0.0, 0.0, 2.0], [1.0, inf, 1.0]]
    idx, valid = _cat(impl, w, [0.7] * 5, device)
    assert valid.tolist() == [False, True, False, True, False]
    assert idx.tolist() == [0, 1, 0, 2, 0]
    assert idx.dtype == torch.int64


def _three_state(impl, device, draft, d, q, p, u_accept=0.5, u_final=0.5, vocab=4):
    w1 = len(draft)
    r = impl.speculative_accept(
        torch.tensor([draft], dtype=torch.int64).to(device),
        torch.tensor([d], dtype=torch.int64).to(device),
        torch.tensor([q], dtype=torch.float32).view(1, w1, vocab).to(device),
        torch.tensor([p], dtype=torch.float32).view(1, w1 + 1, vocab).to(device),
        torch.full((1, w1), u_accept).to(device),
        torch.full((1,), u_final).to(device),
    )
    return r.tokens[0].tolist(), r.accepted.item(), r.final.item(), r.error.item()


def kat_accept_three_state(impl, device):
    assert _three_state(impl, device, [0, 1, 0], 3, [E0, E1, BAD], [E2, E1, E0, E0]) == (
        [2, 0, 0, 0], 0, 2, False)
    tokens, accepted, final, error = _three_state(impl, device, [0, 1, 0], 3, [E0, E1, BAD],
                                                  [E0, E1, E0, E0])
    assert error and accepted == 2 and final == 0 and all(0 <= t < 4 for t in tokens)
    for bonus in ([0.0] * 4, BAD, [float("inf"), 0.0, 0.0, 0.0]):
        assert _three_state(impl, device, [0, 1], 2, [E0, E1], [E0, E1, bonus]) == (
            [0, 1, 0], 2, 0, True)
    for pad in (0, 3, 99, -1):
        assert _three_state(impl, device, [1, pad, pad], 1, [E1, BAD, BAD], [E1, E2, BAD, BAD]) == (
            [1, 2, 0, 0], 1, 2, False)
    for tiny in (1e-38, 1e-30):
        row = [tiny, 1.0, 0.0, 0.0]
        assert _three_state(impl, device, [0], 1, [row], [row, E3], u_accept=BELOW_ONE) == (
            [0, 3], 1, 3, False)


def kat_accept_zero_drafts(impl, device):
    n, vocab = 5, 4
    p = torch.zeros(n, 1, vocab)
    p[torch.arange(n), 0, torch.arange(n) % vocab] = 2.0
    r = impl.speculative_accept(
        torch.zeros(n, 0, dtype=torch.int64).to(device), torch.zeros(n, dtype=torch.int64).to(device),
        torch.zeros(n, 0, vocab).to(device), p.to(device), torch.zeros(n, 0).to(device),
        torch.full((n,), 0.3).to(device))
    assert r.accepted.tolist() == [0] * n
    assert r.final.tolist() == [i % vocab for i in range(n)]
    assert r.tokens.tolist() == [[i % vocab] for i in range(n)]
    assert not r.error.any()


def kat_accept_output_layout(impl, device):
    q = torch.tensor([[E0, E1, E0], [E2, E2, E2], [BAD, BAD, BAD], [BAD, E1, E1], [E0, E0, E0]])
    p = torch.tensor([[E0, E1, E3, E3], [E2, E2, E2, E3], [E1, BAD, BAD, BAD], [E0, E1, E1, E1],
                      [E0, E0, E0, [0.0] * 4]])
    dt = torch.tensor([[0, 1, 0], [2, 2, 2], [0, 0, 0], [0, 1, 1], [0, 0, 0]])
    drafts = torch.tensor([3, 3, 0, 3, 3])
    ua = torch.full((5, 3), 0.5)
    uf = torch.full((5,), 0.5)
    args = [t.to(device) for t in (dt, drafts, q, p, ua, uf)]
    originals = [a.clone() for a in args]
    r = impl.speculative_accept(*args)
    assert r.error.tolist() == [False, False, False, True, True]
    assert r.accepted.tolist() == [2, 3, 0, 0, 3]
    assert r.final.tolist() == [3, 3, 1, 0, 0]
    assert r.tokens.tolist() == [[0, 1, 3, 0], [2, 2, 2, 3], [1, 0, 0, 0], [0, 0, 0, 0], [0, 0, 0, 0]]
    for out in (r.tokens, r.accepted, r.final):
        assert out.dtype == torch.int64
    assert r.error.dtype == torch.bool
    for t, o in zip(args, originals):
        torch.testing.assert_close(t, o, rtol=0, atol=0, equal_nan=True)


def _exact_first_position(impl, device, p0, p1, q, m):
    vocab = len(q)
    qn = [w / sum(q) for w in q]
    xs = [x for x in range(vocab) if qn[x] > 0]
    grid = ((torch.arange(m, dtype=torch.float64) + 0.5) / m).float()
    x_idx = torch.tensor(xs)
    n = len(xs) * m * m
    draft = x_idx.repeat_interleave(m * m)[:, None]
    ua = grid.repeat_interleave(m).repeat(len(xs))[:, None]
    uf = grid.repeat(m * len(xs))
    weight = torch.tensor(qn, dtype=torch.float64)[draft[:, 0]]
    p = torch.tensor([p0, p1], dtype=torch.float32).expand(n, 2, vocab).contiguous()
    qq = torch.tensor(q, dtype=torch.float32).expand(n, 1, vocab).contiguous()
    out = impl.speculative_accept(draft.to(device), torch.ones(n, dtype=torch.int64).to(device),
                                  qq.to(device), p.to(device), ua.to(device), uf.to(device))
    assert not out.error.any()
    tok = out.tokens.cpu()
    acc = (out.accepted.cpu() == 1).double()
    total = float(m * m)
    first = torch.bincount(tok[:, 0], weights=weight, minlength=vocab) / total
    p_acc = (weight * acc).sum() / total
    bonus = torch.bincount(tok[:, 1], weights=weight * acc, minlength=vocab)
    bonus = bonus / (weight * acc).sum().clamp_min(1e-30)
    return first, p_acc.item(), bonus, (weight * acc).sum().item() > 0


EXACT_CASES = {
    "generic": ([0.5, 4.0, 1.0, 0.0, 2.0], [3.0, 1.0, 0.0, 2.0, 6.0], [2.0, 0.0, 1.0, 3.0, 0.5]),
    "disjoint": ([0.0, 0.0, 1.0, 3.0, 2.0], [1.0, 1.0, 2.0, 0.0, 5.0], [1.0, 2.0, 0.0, 0.0, 0.0]),
    "equal": ([2.0, 0.0, 1.0, 3.0, 0.5], [4.0, 1.0, 1.0, 1.0, 1.0], [2.0, 0.0, 1.0, 3.0, 0.5]),
}


def _normalized(w):
    return torch.tensor([x / sum(w) for x in w], dtype=torch.float64)


def kat_accept_exact_quadrature(impl, device):
    m = 256
    for case, (p0, p1, q) in EXACT_CASES.items():
        first, p_acc, bonus, has = _exact_first_position(impl, device, p0, p1, q, m)
        pn0, pn1, qn = _normalized(p0), _normalized(p1), _normalized(q)
        assert (first - pn0).abs().max() <= 3 / m, case
        assert abs(p_acc - torch.minimum(pn0, qn).sum().item()) <= 3 / m, case
        if case == "disjoint":
            assert p_acc == 0
        if case == "equal":
            assert abs(p_acc - 1.0) <= 1e-9
        if has:
            assert (bonus - pn1).abs().max() <= 3 / m, case
    first, *_ = _exact_first_position(impl, device, [3.0, 2.0], [1.0, 1.0], [1.0, 3.0], m)
    assert (first - torch.tensor([0.6, 0.4], dtype=torch.float64)).abs().max() <= 3 / m


ALL_KATS = [
    kat_categorical_midpoint_quadrature,
    kat_categorical_trailing_zeros,
    kat_categorical_out_of_contract_uniform,
    kat_categorical_small_token_after_large_mass,
    kat_categorical_fp64_cdf,
    kat_categorical_exact_boundaries,
    kat_categorical_plateau_tail,
    kat_categorical_invalid_rows,
    kat_accept_three_state,
    kat_accept_zero_drafts,
    kat_accept_output_layout,
    kat_accept_exact_quadrature,
]
