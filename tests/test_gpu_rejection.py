"""Synchronous runner's rejection sampling on gfx950 (vllm_rlt/worker/speculative.py:56-72,
574-625): kernel decisions and residual rows bit-exact with the torch-CPU oracle, the
generator protocol against the reference loop run on the device, the error cases, and
the reference's distribution-recovery test."""

import sys

import pytest
import torch

from oracle import sampling as osamp

pytestmark = pytest.mark.gpu


def _say(*args):
    print("[case]", *args, flush=True)
    sys.stdout.flush()


def _inputs(n, k, vocab, g, temperature=1.0, top_p=1.0, noise=1.0):
    dl = torch.randn(n, k + 1, vocab, generator=g) * 3
    tl = dl + torch.randn(n, k + 1, vocab, generator=g) * noise
    rows = lambda x: osamp.batched_probabilities(  # noqa: E731
        x.reshape(-1, vocab), torch.full((x.shape[0] * x.shape[1],), temperature),
        torch.full((x.shape[0] * x.shape[1],), -1, dtype=torch.int64),
        torch.full((x.shape[0] * x.shape[1],), top_p), max_top_k=0,
        apply_top_p=top_p < 1).view(x.shape)
    q = rows(dl[:, :k].contiguous())
    p = rows(tl)
    u = torch.rand(n, k, generator=g)
    cand = torch.stack([osamp.categorical(q[:, j], torch.rand(n, generator=g))[0]
                        for j in range(k)], 1)
    return p, q, u, cand


def _oracle_rows(cand, counts, p, q, u):
    """Per request: (status, accepted, normalized residual or None) from rejection_step."""
    out = []
    for i in range(cand.shape[0]):
        res = (0, int(counts[i]), None)
        for j in range(int(counts[i])):
            c = int(cand[i, j])
            if c < -p.shape[-1] or c >= p.shape[-1]:
                res = (4, j, None)
                break
            try:
                ok, r = osamp.rejection_step(c, p[i, j], q[i, j], u[i, j])
            except ValueError:
                res = (2, j, None)
                break
            except RuntimeError:
                res = (3, j, None)
                break
            if not ok:
                res = (1, j, r)
                break
        out.append(res)
    return out


def _check_rows(pkg, dev, cand, counts, p, q, u, threads):
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        want = _oracle_rows(cand, counts, p, q, u)
    finally:
        torch.set_num_threads(prev)
    status, accepted, residual = pkg.sampling.rejection_rows(
        cand.to(dev), counts.to(dev), p.to(dev), q.to(dev), u.to(dev), sum_threads=threads)
    status, accepted, residual = status.cpu(), accepted.cpu(), residual.cpu()
    for i, (st, a, r) in enumerate(want):
        assert (int(status[i]), int(accepted[i])) == (st, a), f"request {i}"
        if st == 1:
            assert torch.equal(residual[i], r), f"request {i} residual"
    return want


@pytest.mark.parametrize("name,n,vocab,temperature,top_p,threads", [
    ("config1", 8, 49152, 1.0, 1.0, 1),
    ("config1", 8, 49152, 1.0, 1.0, 16),
    ("config3", 32, 49152, 0.7, 0.9, 4),
    ("config5", 64, 65536, 1.0, 1.0, 16),
    ("wide", 6, 151936, 1.0, 1.0, 5),
    ("small", 16, 1000, 1.0, 1.0, 8),
])
def test_rejection_rows_bit_exact(pkg, dev, name, n, vocab, temperature, top_p, threads):
    _say("rejection rows", name, threads)
    g = torch.Generator().manual_seed(vocab + n + threads)
    k = 4
    p, q, u, cand = _inputs(n, k, vocab, g, temperature, top_p)
    counts = torch.randint(0, k + 1, (n,), generator=g)
    counts[0] = k
    want = _check_rows(pkg, dev, cand, counts, p, q, u, threads)
    assert sum(st == 1 for st, _, _ in want) >= n // 4  # rejections were exercised


def test_rejection_rows_error_cases(pkg, dev):
    _say("rejection errors")
    g = torch.Generator().manual_seed(9)
    n, k, vocab = 6, 4, 3000
    p, q, u, cand = _inputs(n, k, vocab, g, noise=0.01)
    counts = torch.full((n,), k)
    q[0, 1, cand[0, 1]] = 0.0                      # zero proposal mass at draft 1
    cand[1, 0] = vocab                             # out of the vocabulary
    cand[2, 2] = -5                                # negative ids index from the end
    u[3] = 0.999999                                # force a rejection ...
    p[3, 0] = q[3, 0]                              # ... with a zero residual is impossible
    p[3, 0, 7] = float("nan")                      # a NaN total instead
    q[3, 0, cand[3, 0]] = 1.0
    q[4, 2, cand[4, 2]] = float("nan")             # NaN proposal mass
    want = _check_rows(pkg, dev, cand, counts, p, q, u, 4)
    st = [w[0] for w in want]
    assert st[1] == 4 and st[3] == 3 and 2 in (st[0], st[4])


def _generators(n, dev, seed):
    return [torch.Generator(device=dev).manual_seed(seed + i) for i in range(n)]


def _ulps(a, b):
    """Distance in float32 units in the last place between two positive floats."""
    ia = torch.tensor([a], dtype=torch.float32).view(torch.int32).item()
    ib = torch.tensor([b], dtype=torch.float32).view(torch.int32).item()
    return abs(ia - ib)


@pytest.mark.parametrize("seed", [21, 22, 23, 24])
def test_rejection_round_against_the_reference_loop_on_the_device(pkg, dev, seed):
    """The reference loop run on the device (vllm_rlt/worker/speculative.py:56-72 under
    :574-625) normalizes the residual by torch-ROCm's ``residual.sum()``; the kernels use
    one fixed order (torch's single-thread CPU order, ``sum_threads=1``).  The accept
    decisions involve no sum and must agree for every request; the generator protocol
    (every generator's final state) must agree too.  A request's tokens may differ only
    after a rejection whose residual totals differ -- by at most a few float32 ulps, the
    spread of two summation orders over V terms -- and every request whose totals agree
    bit for bit must draw the same token."""
    _say("rejection round vs device loop", seed)
    g = torch.Generator().manual_seed(seed)
    n, k, vocab = 32, 4, 49152
    p, q, u, cand = _inputs(n, k, vocab, g, temperature=0.7, top_p=0.9)
    counts = torch.randint(0, k + 1, (n,), generator=g).tolist()
    cands = [cand[i, :counts[i]].tolist() for i in range(n)]
    pd, qd = p.to(dev), q.to(dev)
    ours_g, ref_g = _generators(n, dev, 100 + seed), _generators(n, dev, 100 + seed)
    got = pkg.sampling.rejection_round(cands, pd, qd, ours_g)
    want = osamp.collect_stochastic(cands, pd, qd, ref_g)
    for a, b in zip(ours_g, ref_g):
        assert torch.equal(a.get_state(), b.get_state())
    prev = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        differing = 0
        for i, ((tok_a, acc_a), (tok_b, acc_b)) in enumerate(zip(got, want)):
            assert acc_a == acc_b, f"request {i}: accept decisions differ"
            if acc_a == len(cands[i]):
                assert tok_a == tok_b, f"request {i}: bonus draw from the same p row"
                continue
            residual = (p[i, acc_a] - q[i, acc_a]).clamp_min(0)
            ours = residual.sum().item()  # the kernels' order (pinned against them)
            device = (pd[i, acc_a] - qd[i, acc_a]).clamp_min(0).sum().item()
            if ours == device:
                assert tok_a == tok_b, f"request {i}: equal totals, different draws"
            elif tok_a != tok_b:
                differing += 1
                assert _ulps(ours, device) <= 8, f"request {i}: totals {ours} vs {device}"
    finally:
        torch.set_num_threads(prev)
    assert differing <= 2
    assert sum(a < len(c) for (_, a), c in zip(got, cands)) >= 4  # rejections happened


def test_rejection_round_error_leaves_generators_as_the_reference(pkg, dev):
    _say("rejection round error")
    g = torch.Generator().manual_seed(22)
    n, k, vocab = 4, 4, 2000
    p, q, u, cand = _inputs(n, k, vocab, g, noise=0.001)  # nearly always accepted
    cands = [cand[i].tolist() for i in range(n)]
    q[1, 2, cands[1][2]] = 0.0  # request 1 fails at draft 2 unless it stops earlier
    pd, qd = p.to(dev), q.to(dev)
    ours_g, ref_g = _generators(n, dev, 7), _generators(n, dev, 7)
    err = None
    try:
        osamp.collect_stochastic(cands, pd, qd, ref_g)
    except ValueError as e:
        err = e
    if err is None:
        pytest.skip("request 1 stopped before its zero-mass draft on this seed")
    with pytest.raises(ValueError):
        pkg.sampling.rejection_round(cands, pd, qd, ours_g)
    for a, b in zip(ours_g, ref_g):
        assert torch.equal(a.get_state(), b.get_state())


def test_rejection_sample_single_draft_matches_reference(pkg, dev):
    _say("rejection single")
    g = torch.Generator().manual_seed(23)
    p, q, u, cand = _inputs(16, 1, 49152, g)
    for i in range(16):
        a, b = torch.Generator(device=dev).manual_seed(i), torch.Generator(device=dev).manual_seed(i)
        x = int(cand[i, 0])
        pd, qd = p[i, 0].to(dev), q[i, 0].to(dev)
        got = pkg.sampling.rejection_sample(x, pd, qd, a)
        want = osamp.rejection_sample(x, pd, qd, b)
        assert got[1] == want[1] and torch.equal(a.get_state(), b.get_state())
        if got[0] != want[0]:
            # only a residual draw whose totals differ (the reference's is torch-ROCm's)
            residual = (p[i, 0] - q[i, 0]).clamp_min(0)
            prev = torch.get_num_threads()
            torch.set_num_threads(1)
            ours = residual.sum().item()
            torch.set_num_threads(prev)
            device = (pd - qd).clamp_min(0).sum().item()
            assert not got[1] and ours != device and _ulps(ours, device) <= 8
    # zero proposal mass: raises before drawing, the generator untouched
    qz = q[0, 0].clone()
    qz[int(cand[0, 0])] = 0
    a = torch.Generator(device=dev).manual_seed(5)
    before = a.get_state()
    with pytest.raises(ValueError):
        pkg.sampling.rejection_sample(int(cand[0, 0]), p[0, 0].to(dev), qz.to(dev), a)
    assert torch.equal(a.get_state(), before)


@pytest.mark.parametrize("p,q", [
    ([0.1, 0.6, 0.3], [0.7, 0.2, 0.1]),
    ([0.0, 1.0, 0.0], [1.0, 0.0, 0.0]),
    ([0.2, 0.3, 0.5], [0.2, 0.3, 0.5]),
])
def test_rejection_sample_recovers_target_distribution(pkg, dev, p, q):
    # reference known answer: tests/test_speculative.py:455-471, on the device
    _say("rejection recovery", p, q)
    p, q = torch.tensor(p, device=dev), torch.tensor(q, device=dev)
    g = torch.Generator(device=dev).manual_seed(431)
    counts = torch.zeros(3)
    for _ in range(12000):
        candidate = int(torch.multinomial(q, 1, generator=g))
        token, _ = pkg.sampling.rejection_sample(candidate, p, q, g)
        counts[token] += 1
    torch.testing.assert_close(counts / counts.sum(), p.cpu(), atol=0.016, rtol=0)
