"""gfx950 sampling distributions (batched_probabilities) and the device greedy round.

Parity bar: probabilities within atol 1e-6 / rtol 1e-5 of the torch-CPU oracle (the
tolerance of the reference's own test, tests/test_speculative_sampling.py:44-60).
The top-p cut is pinned to exact arithmetic: the kernel decides it on exact
fixed-point sums of its token masses, and its kept count must equal the float64 cut
up to tokens within 2e-6 of the threshold (the masses' own error).  torch's float32 softmax sums
to 1 + d (|d| ~ 1e-5 at V = 65536), so its own cut may differ from the exact one by a
few tail tokens; the support may differ from the oracle's only there.  Tokens tied at a top-k / top-p cut survive in column
order on the GPU; the reference leaves that choice unspecified, so tie cases are
checked by count and value.  The greedy round (argmax + prefix match) is bit-exact.
"""

import sys
import zlib

import pytest
import torch

from oracle import sampling as osamp

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-6, 1e-5
# the kernel's token masses (hardware exp2 of (l - lmax) log2(e) / T) carry ~1e-6
# relative error, so its cut equals the float64 one except within this band
EXACT_BAND = 2e-6


def _say(*args):
    print("[case]", *args, flush=True)
    sys.stdout.flush()


def _host_args(top_k, top_p, vocab):
    # reference: tests/test_speculative_sampling.py:15-21
    eff = [int(k) for k in top_k if 0 < int(k) < vocab]
    return {"max_top_k": max(eff, default=0), "apply_top_p": any(float(p) < 1 for p in top_p)}


def _run(pkg, dev, logits, temperature, top_k, top_p, **plan):
    vocab = logits.shape[-1]
    t = torch.as_tensor(temperature, dtype=torch.float32)
    k = torch.as_tensor(top_k, dtype=torch.int64)
    p = torch.as_tensor(top_p, dtype=torch.float32)
    plan = plan or _host_args(k.tolist(), p.tolist(), vocab)
    got = pkg.batched_probabilities(logits.to(dev), t.to(dev), k.to(dev), p.to(dev), **plan).cpu()
    want = osamp.batched_probabilities(logits, t, k, p, **plan)
    return got, want, t, k, p, plan


def _filtered_logits(logits_row, t, k, plan):
    """x = logits / T after the reference's top-k step (torch, as the oracle)."""
    x = logits_row.float() / t
    vocab = x.shape[-1]
    if plan["max_top_k"] > 0 and 0 < k < vocab:
        vals, idx = x.topk(min(k, plan["max_top_k"]))
        x = torch.full_like(x, -torch.inf).scatter_(0, idx, vals)
    return x


def _exact_kept(sx, top_p):
    """Top-p kept count of a descending row in float64 (the exact decision the kernel's
    fixed-point masses reproduce), with the preceding mass of every position."""
    fin = torch.isfinite(sx)
    e = torch.zeros(sx.shape, dtype=torch.float64)
    e[fin] = (sx[fin].double() - sx[0].double()).exp()
    before = (e.cumsum(0) - e) / e.sum()
    kept = max(1, int((before <= top_p).sum()))
    return min(kept, int(fin.sum()) if top_p > 0 else 1), before


def _assert_match(got, want, logits, t, k, p, plan):
    """Tie-invariant comparison.

    * The kept set must be a top set of x (as a multiset of values).
    * Rows with top-p: its size must equal the float64 exact cut (up to positions
      whose preceding mass is within EXACT_BAND of p), and may differ from torch's only at
      positions within torch's own error: its fp32 softmax sums to 1 + d, |d| up to
      ~1e-5 at V = 65536, which shifts every cumulative value it compares with p.
    * Probabilities match position by position when the supports agree, else as
      sorted values (tied tokens permuted)."""
    assert got.dtype == torch.float32 and got.shape == want.shape
    for i in range(got.shape[0]):
        g, w = got[i], want[i]
        gs, ws = g > 0, w > 0
        x = _filtered_logits(logits[i], t[i], int(k[i]), plan)
        sx = x.sort(descending=True).values
        gc, wc = int(gs.sum()), int(ws.sum())
        top_p = float(p[i])
        if plan["apply_top_p"] and top_p < 1 and bool(torch.isfinite(sx[0])):
            ec, before = _exact_kept(sx, top_p)
            if gc != ec:
                lo, hi = min(gc, ec), max(gc, ec)
                assert ((before[lo:hi] - top_p).abs() <= EXACT_BAND).all(), f"row {i}: {gc} vs exact {ec}"
        if torch.equal(gs, ws):
            torch.testing.assert_close(g, w, atol=ATOL, rtol=RTOL)
            continue
        assert torch.equal(x[gs].sort(descending=True).values, sx[:gc]), f"row {i}: not a top set"
        if gc != wc:
            assert plan["apply_top_p"] and top_p < 1, f"row {i}: {gc} vs {wc} kept"
            sm = sx.softmax(-1)
            band = 2 * abs(sm.double().sum().item() - 1) + 1e-6
            tb = sm.cumsum(-1) - sm
            lo, hi = min(gc, wc), max(gc, wc)
            assert ((tb[lo:hi] - top_p).abs() <= band).all(), f"row {i}: {gc} vs torch {wc}"
            # torch's kept set is a top set too, so the two differ only by tail positions
            # lo..hi of the order (tied tokens may be swapped, which leaves the values).
            assert torch.equal(x[ws].sort(descending=True).values, sx[:wc]), \
                f"row {i}: torch's kept set is not a top set"
            # Values: both rows renormalised over the common support agree token by token.
            common = gs & ws
            gn = g[common].double() / g[common].double().sum()
            wn = w[common].double() / w[common].double().sum()
            torch.testing.assert_close(gn, wn, atol=ATOL, rtol=RTOL)
            # And before renormalising, each side's kept mass over the common support is
            # 1 minus its extra tail tokens' mass.
            torch.testing.assert_close(g[common].double().sum() + g[gs & ~ws].double().sum(),
                                       torch.tensor(1.0, dtype=torch.float64), atol=1e-5, rtol=0)
            continue
        torch.testing.assert_close(g.sort().values, w.sort().values, atol=ATOL, rtol=RTOL)


# ------------------------------------------------------------ reference known answers

def test_closed_form_filters(pkg, dev):
    # reference: tests/test_speculative.py:474-490
    _say("closed forms")
    logits = torch.tensor([[0.50, 0.25, 0.15, 0.10]]).log()
    got, *_ = _run(pkg, dev, logits, [1.0], [-1], [0.8])
    torch.testing.assert_close(got[0], torch.tensor([0.50, 0.25, 0.15, 0]) / 0.9)
    got, *_ = _run(pkg, dev, logits, [0.5], [2], [1.0])
    torch.testing.assert_close(got[0], torch.tensor([0.8, 0.2, 0, 0]))
    got, *_ = _run(pkg, dev, torch.zeros(1, 4), [1.0], [1], [1.0])
    assert int((got > 0).sum()) == 1
    torch.testing.assert_close(got[got > 0], torch.ones(1))


def test_matches_row_by_row_sampler(pkg, dev):
    # reference: tests/test_speculative_sampling.py:44-60
    _say("row-by-row matrix")
    vocab = 17
    g = torch.Generator().manual_seed(0)
    top_ks = [-1, 1, 3, vocab, vocab + 5]
    top_ps = [1.0, 0.9, 0.5]
    temps = [0.5, 0.8, 1.0, 1.5, 2.0]
    tk = [top_ks[i % 5] for i in range(30)]
    tp = [top_ps[(i // 5) % 3] for i in range(30)]
    tt = [temps[(i * 3) % 5] for i in range(30)]
    logits = torch.randn(30, vocab, generator=g) * 3
    got, want, t, k, p, plan = _run(pkg, dev, logits, tt, tk, tp)
    rows = torch.stack([osamp.sampler_probabilities(logits[i], tt[i], tk[i], tp[i])
                        for i in range(30)])
    torch.testing.assert_close(want, rows, atol=ATOL, rtol=RTOL)
    _assert_match(got, want, logits, t, k, p, plan)
    torch.testing.assert_close(got.sum(-1), torch.ones(30), atol=1e-6, rtol=0)


def test_top_k_is_strict_with_ties(pkg, dev):
    # reference: tests/test_speculative_sampling.py:63-86
    _say("strict top-k ties")
    got, *_ = _run(pkg, dev, torch.tensor([[5.0, 4.0, 4.0, 1.0]]), [1.0], [2], [1.0])
    probs = got[0]
    assert (probs > 0).sum().item() == 2 and probs[0] > 0 and probs[3] == 0
    assert (probs[1] > 0) != (probs[2] > 0)
    kept = 1 if probs[1] > 0 else 2
    torch.testing.assert_close(probs[[0, kept]], torch.tensor([5.0, 4.0]).softmax(-1))
    got, *_ = _run(pkg, dev, torch.zeros(1, 6), [1.0], [2], [1.0])
    assert (got[0] > 0).sum().item() == 2


def test_top_p_one_row_keeps_full_support(pkg, dev):
    # reference: tests/test_speculative_sampling.py:89-99
    _say("top_p = 1 next to top_p < 1")
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(2, 64, generator=g) * 2
    got, want, t, k, p, plan = _run(pkg, dev, logits, [1.0, 1.0], [-1, -1], [1.0, 0.5])
    assert (got[0] > 0).all() and (got[1] > 0).sum() < 64
    torch.testing.assert_close(got[0], logits[0].softmax(-1), atol=ATOL, rtol=RTOL)
    _assert_match(got, want, logits, t, k, p, plan)


# ------------------------------------------------------------ seeded parity

@pytest.mark.parametrize("name,n,vocab,temperature,top_p,dtype", [
    ("config1-q", 32, 49152, 1.0, 1.0, torch.float32),
    ("config3-p", 160, 49152, 0.7, 0.9, torch.float32),
    ("config3-bf16", 64, 49152, 0.7, 0.9, torch.bfloat16),
    ("config4", 40, 65536, 1.0, 1.0, torch.float32),
    ("config5-p", 40, 65536, 1.0, 0.9, torch.float16),
])
def test_config_shaped_parity(pkg, dev, name, n, vocab, temperature, top_p, dtype):
    _say("config", name)
    g = torch.Generator().manual_seed(zlib.crc32(name.encode()))
    logits = (torch.randn(n, vocab, generator=g) * 3).to(dtype)
    got, want, t, k, p, plan = _run(pkg, dev, logits, [temperature] * n, [-1] * n, [top_p] * n)
    _assert_match(got, want, logits, t, k, p, plan)


@pytest.mark.parametrize("vocab", [1, 2, 17, 1000, 1024, 1025, 4096, 4097, 16384, 16385, 32768,
                                   32769, 49152, 49153, 57344, 59000, 61440, 65536, 65537, 128256, 131072 + 3, 151936])
def test_mixed_filters_across_vocab_sizes(pkg, dev, vocab):
    """Every row placement (registers, registers + LDS, re-reading) with a mix of
    temperatures, top-k (including k >= V and k <= 0) and top-p per row."""
    _say("mixed filters V", vocab)
    g = torch.Generator().manual_seed(vocab)
    n = 12
    logits = torch.randn(n, vocab, generator=g) * torch.tensor([0.5, 2, 4, 8] * 3)[:, None]
    tt = [0.5, 0.7, 1.0, 1.3, 2.0, 0.9, 1.0, 0.6, 1.1, 0.8, 1.0, 3.0]
    tk = [-1, 1, 5, 40, vocab, vocab + 3, 0, 1000, 7, -1, 2, 300]
    tp = [1.0, 0.9, 0.5, 0.95, 0.3, 1.0, 0.99, 0.9, 0.0, 0.999, 0.6, 0.8]
    got, want, t, k, p, plan = _run(pkg, dev, logits, tt, tk, tp)
    _assert_match(got, want, logits, t, k, p, plan)


def test_inconsistent_plan_follows_reference(pkg, dev):
    """max_top_k below a row's k keeps max_top_k tokens; apply_top_p=False skips top-p
    for every row (reference: speculative_sampling.py:39-55)."""
    _say("host plan semantics")
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(4, 5000, generator=g) * 2
    got, want, t, k, p, plan = _run(pkg, dev, logits, [1.0] * 4, [50, 10, -1, 4000],
                                    [0.5, 0.9, 0.7, 1.0], max_top_k=20, apply_top_p=False)
    assert [(got[i] > 0).sum().item() for i in range(4)] == [20, 10, 5000, 20]
    _assert_match(got, want, logits, t, k, p, plan)


def test_ties_and_degenerate_rows(pkg, dev):
    _say("ties / -inf / NaN rows")
    vocab = 6000
    logits = torch.zeros(6, vocab)
    logits[1, ::2] = -torch.inf                 # masked vocabulary, k beyond the finite count
    logits[2, :3] = 4.0                          # three-way tie at the top
    logits[3] = torch.arange(vocab) % 7          # large tie groups
    logits[4, 17] = float("nan")                 # NaN row
    logits[5, :] = -torch.inf                    # no finite logit
    tk = [3, 4000, 2, 1000, -1, -1]
    tp = [0.45, 1.0, 1.0, 0.5, 0.9, 0.9]
    got, want, *_ = _run(pkg, dev, logits, [1.0] * 6, tk, tp)
    # row 0: uniform; top-k keeps 3, top-p 0.45 then keeps the two whose preceding
    # mass (0, 1/3) is <= 0.45
    assert (got[0] > 0).sum().item() == 2
    torch.testing.assert_close(got[0][got[0] > 0], torch.full((2,), 0.5))
    # row 1: 3000 finite zeros survive top-k 4000 (the -inf picks carry no mass)
    assert (got[1] > 0).sum().item() == 3000
    torch.testing.assert_close(got[1][got[1] > 0], torch.full((3000,), 1 / 3000))
    # row 2: exactly two of the three tied maxima, in column order on the GPU
    assert (got[2] > 0).sum().item() == 2 and got[2, 0] > 0 and got[2, 1] > 0
    # row 3: top-k 1000 keeps the 857 sixes and 143 fives; top-p 0.5 ends inside the
    # sixes: floor(0.5 (857 + 143 / e)) + 1 = 455 of them, as many as torch keeps
    assert (got[3] > 0).sum().item() == 455 == (want[3] > 0).sum().item()
    assert (got[3] > 0).nonzero().flatten().tolist() == list(range(6, 7 * 455, 7))
    assert torch.isnan(got[4]).all() and torch.isnan(got[5]).all()


def test_strided_logits_and_inputs_unchanged(pkg, dev):
    _say("strided logits")
    g = torch.Generator().manual_seed(11)
    big = torch.randn(8, 3000, generator=g).to(dev)
    view = big[:, 100:2148]                      # row stride 3000, V = 2048
    snap = big.clone()
    t = torch.full((8,), 0.8, device=dev)
    k = torch.full((8,), 50, dtype=torch.int64, device=dev)
    p = torch.full((8,), 0.9, device=dev)
    got = pkg.batched_probabilities(view, t, k, p, max_top_k=50, apply_top_p=True).cpu()
    want = osamp.batched_probabilities(view.cpu(), t.cpu(), k.cpu(), p.cpu(), max_top_k=50,
                                       apply_top_p=True)
    assert torch.equal(big, snap)
    _assert_match(got, want, view.cpu(), t.cpu(), k.cpu(), p.cpu(),
                  {"max_top_k": 50, "apply_top_p": True})


def test_shape_errors(pkg, dev):
    x = torch.zeros(3, 10, device=dev)
    t = torch.ones(3, device=dev)
    k = torch.zeros(3, dtype=torch.int64, device=dev)
    with pytest.raises(ValueError):
        pkg.batched_probabilities(x[0], t, k, t, max_top_k=0, apply_top_p=False)
    with pytest.raises(ValueError):
        pkg.batched_probabilities(x, t[:2], k, t, max_top_k=0, apply_top_p=False)
    with pytest.raises(ValueError):
        pkg.batched_probabilities(x, t, k, t, max_top_k=-1, apply_top_p=False)


# ------------------------------------------------------------ greedy round

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("vocab", [5, 1000, 49152, 65536])
def test_greedy_round_bit_exact(pkg, dev, dtype, vocab):
    _say("greedy", dtype, vocab)
    g = torch.Generator().manual_seed(vocab)
    n, w1 = 48, 4
    logits = torch.randn(n, w1 + 1, vocab, generator=g).to(dtype)
    # integer logits on some rows force ties (first column must win); NaN rows win at NaN
    logits[::5] = torch.randint(0, 3, (len(range(0, n, 5)), w1 + 1, vocab), generator=g).to(dtype)
    logits[7, 2, vocab // 2] = float("nan")
    logits[7, 2, vocab - 1] = float("nan")
    targets = logits.float().argmax(-1)
    draft = torch.where(torch.rand(n, w1, generator=g) < 0.75, targets[:, :w1],
                        torch.randint(0, vocab, (n, w1), generator=g))
    drafts = torch.randint(0, w1 + 1, (n,), generator=g)
    want = osamp.greedy_accept_batched(draft, drafts, logits.float())
    got = pkg.greedy_accept_batched(draft.to(dev), drafts.to(dev), logits.to(dev))
    for a, b in zip(got, want):
        assert torch.equal(a.cpu(), b)
    assert got[0][7, 2].item() == vocab // 2


@pytest.mark.parametrize("vocab", [3000, 49152, 57000, 59000, 61000, 65536, 100003])
def test_crowded_rows_use_the_exact_path(pkg, dev, vocab):
    """Near-flat rows put thousands of tokens into one mass bin, more than the fast
    kernel's sorted list holds: those rows are recomputed by the exact path, the
    others in the same call stay on the fast path."""
    _say("crowded rows V", vocab)
    g = torch.Generator().manual_seed(vocab + 1)
    n = 6
    logits = torch.randn(n, vocab, generator=g)
    logits[0] *= 1e-3                     # flat: top-p cut inside one crowded bin
    logits[1] *= 1e-3                     # flat: top-k cut inside one crowded bin
    logits[2] = torch.floor(logits[2] * 2) / 2   # few distinct values, large tie groups
    logits[3] *= 4                        # ordinary rows
    logits[4] *= 4
    logits[5] *= 1e-3
    tt = [1.0, 1.0, 1.0, 0.7, 0.7, 1.0]
    tk = [-1, vocab // 3, vocab // 2, -1, 40, vocab // 4]
    tp = [0.5, 1.0, 0.3, 0.9, 0.95, 0.6]
    got, want, t, k, p, plan = _run(pkg, dev, logits, tt, tk, tp)
    _assert_match(got, want, logits, t, k, p, plan)
    assert (got[1] > 0).sum().item() == vocab // 3


# ------------------------------------------------------------ draft proposals

@pytest.mark.parametrize("dtype,vocab", [(torch.float32, 49152), (torch.bfloat16, 5000),
                                         (torch.float16, 65536), (torch.bfloat16, 20000),
                                         (torch.float32, 12289), (torch.float16, 4099)])
def test_propose_drafts_matches_reference_composition(pkg, dev, dtype, vocab):
    """async_speculative.py:645-663: argmax for every drafting row, random rows
    replaced by categorical(q_o, u); q_o written into the q[:, offset] view (a NaN row,
    and a flat row whose top-k cut takes the exact path)."""
    _say("propose_drafts", dtype, vocab)
    g = torch.Generator().manual_seed(vocab)
    m = 12
    logits = (torch.randn(m, vocab, generator=g) * 3).to(dtype)
    logits[5, 17] = float("nan")  # a NaN row: argmax picks the NaN, its q row is NaN
    logits[9] = 1.0  # a flat row: its top-k cut takes the exact path
    random_rows = torch.tensor([0, 3, 4, 5, 9, 11])
    r = len(random_rows)
    t = torch.tensor([0.7, 1.0, 0.5, 1.0, 1.3, 0.9])
    k = torch.tensor([-1, 40, 0, -1, 7, -1])
    p = torch.tensor([0.9, 1.0, 0.8, 1.0, 1.0, 0.95])
    u = torch.rand(r, generator=g)
    plan = _host_args(k.tolist(), p.tolist(), vocab)
    q = torch.full((r, 4, vocab), -1.0, device=dev)
    offset = 2
    proposed, q_o = pkg.propose_drafts(logits.to(dev), random_rows.to(dev), t.to(dev), k.to(dev),
                                       p.to(dev), u.to(dev), q_out=q[:, offset], **plan)
    assert q_o.data_ptr() == q[:, offset].data_ptr()
    got_q = q[:, offset].cpu()
    assert bool((q[:, :offset] == -1).all()) and bool((q[:, offset + 1:] == -1).all())
    want_q = osamp.batched_probabilities(logits[random_rows], t, k, p, **plan)
    good = [i for i in range(r) if int(random_rows[i]) != 5]
    _assert_match(got_q[good], want_q[good], logits[random_rows][good], t[good], k[good],
                  p[good], plan)
    assert torch.isnan(got_q[3]).all()
    # tokens: greedy rows are the argmax; random rows the bit-exact categorical of the
    # q the kernel produced (invalid rows propose token 0)
    want = logits.float().argmax(-1)
    sampled, _ = osamp.categorical(got_q, u)
    want[random_rows] = sampled
    assert torch.equal(proposed.cpu(), want)


def test_propose_drafts_greedy_only_and_bad_rows(pkg, dev):
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(7, 3000, generator=g)
    proposed, q_o = pkg.propose_drafts(logits.to(dev), None, None, None, None, None,
                                       max_top_k=0, apply_top_p=False)
    assert q_o.shape == (0, 3000)
    assert torch.equal(proposed.cpu(), logits.argmax(-1))
    # a random row index outside the batch: NaN q row, no proposal written for it
    rows = torch.tensor([1, 9])
    ones = torch.ones(2)
    proposed, q_o = pkg.propose_drafts(logits.to(dev), rows.to(dev), ones.to(dev),
                                       torch.full((2,), -1).to(dev), ones.to(dev),
                                       torch.full((2,), 0.5).to(dev), max_top_k=0,
                                       apply_top_p=False)
    assert torch.isnan(q_o[1]).all().item()
    want = logits.argmax(-1)
    want[1] = osamp.categorical(q_o[:1].cpu(), torch.full((1,), 0.5))[0][0]
    assert torch.equal(proposed.cpu(), want)


@pytest.mark.parametrize("dtype,vocab", [(torch.bfloat16, 65536), (torch.float32, 50001),
                                         (torch.float16, 151936), (torch.bfloat16, 262144)])
def test_propose_drafts_unfiltered_draws_match_categorical(pkg, dev, dtype, vocab):
    """async_speculative.py:645-663 without top-k/top-p: the row-split distributions
    write the draws' tile totals themselves; the tokens are still torch's categorical
    of the q rows written (ragged last tile, NaN row, row outside the batch)."""
    _say("propose_drafts unfiltered", dtype, vocab)
    g = torch.Generator().manual_seed(vocab + 7)
    m = 9
    logits = (torch.randn(m, vocab, generator=g) * 2).to(dtype)
    logits[4, vocab - 1] = float("nan")
    logits[6] = 0.0  # uniform row
    random_rows = torch.tensor([0, 2, 4, 6, 8, 11, 1])
    r = len(random_rows)
    t = torch.tensor([0.8, 1.0, 1.0, 1.0, 0.6, 1.0, 1.4])
    u = torch.rand(r, generator=g)
    u[3] = 0.5  # exact halfway of the uniform row
    u[6] = 0.0
    ones = torch.ones(r)
    q = torch.full((r, 3, vocab), -1.0, device=dev)  # written through the q[:, 1] view
    proposed, q_o = pkg.propose_drafts(logits.to(dev), random_rows.to(dev), t.to(dev),
                                       torch.full((r,), -1).to(dev), ones.to(dev), u.to(dev),
                                       q_out=q[:, 1], max_top_k=0, apply_top_p=False)
    assert bool((q[:, 0] == -1).all()) and bool((q[:, 2] == -1).all())
    got_q = q[:, 1].cpu()
    assert torch.isnan(got_q[2]).all() and torch.isnan(got_q[5]).all()
    ok = [0, 1, 3, 4, 6]
    x = logits[random_rows[ok]].float() / t[ok, None]
    want_q = osamp.batched_probabilities(logits[random_rows[ok]], t[ok], torch.full((5,), -1),
                                         torch.ones(5), max_top_k=0, apply_top_p=False)
    # the kernel's total is float64: within 5e-6 of the float64 softmax of x = l / T;
    # torch's float32 softmax (the oracle) itself drifts ~6e-11 V relative (1.6e-5 at
    # V = 262144, measured against float64), so the oracle bound widens with V
    torch.testing.assert_close(got_q[ok].double(), torch.softmax(x.double(), -1),
                               rtol=5e-6, atol=1e-12)
    torch.testing.assert_close(got_q[ok], want_q, rtol=max(RTOL, 1e-10 * vocab), atol=ATOL)
    want = logits.float().argmax(-1)
    sampled, _ = osamp.categorical(got_q, u)
    for i, row in enumerate(random_rows.tolist()):
        if row < m:
            want[row] = sampled[i]
    assert torch.equal(proposed.cpu(), want)


def test_propose_drafts_unfiltered_many_random_rows(pkg, dev):
    """More random rows than an argmax slice scans (1024): every greedy row's argmax is
    computed, the random rows' tokens are the categorical of their q rows."""
    _say("propose_drafts unfiltered, 1100 random rows of 1200")
    g = torch.Generator().manual_seed(1200)
    m, vocab = 1200, 4096
    logits = torch.randn(m, vocab, generator=g) * 2
    random_rows = torch.randperm(m, generator=g)[:1100]
    r = len(random_rows)
    t = torch.rand(r, generator=g) + 0.5
    u = torch.rand(r, generator=g)
    ones = torch.ones(r)
    proposed, q_o = pkg.propose_drafts(logits.to(dev), random_rows.to(dev), t.to(dev),
                                       torch.full((r,), -1).to(dev), ones.to(dev), u.to(dev),
                                       max_top_k=0, apply_top_p=False)
    want = logits.argmax(-1)
    want[random_rows] = osamp.categorical(q_o.cpu(), u)[0]
    assert torch.equal(proposed.cpu(), want)


@pytest.mark.parametrize("dtype,vocab", [(torch.float32, 49152), (torch.bfloat16, 3001)])
def test_verify_distributions_match_argmax_and_probabilities(pkg, dev, dtype, vocab):
    """async_speculative.py:678-692: argmax of every verify row, distributions of the
    random rows; bitwise what batched_probabilities gives for the gathered rows."""
    _say("verify distributions", dtype, vocab)
    g = torch.Generator().manual_seed(vocab + 1)
    m = 10
    logits = (torch.randn(m, vocab, generator=g) * 3).to(dtype)
    logits[2, 5] = float("nan")
    rows = torch.tensor([9, 0, 2, 4])
    t = torch.tensor([0.7, 1.0, 0.9, 1.2])
    k = torch.tensor([-1, 30, -1, 0])
    p = torch.tensor([0.9, 1.0, 0.8, 0.95])
    plan = _host_args(k.tolist(), p.tolist(), vocab)
    ld = logits.to(dev)
    out = torch.full((4, 3, vocab), -1.0, device=dev)
    target, p_o = pkg.verify_distributions(ld, rows.to(dev), t.to(dev), k.to(dev), p.to(dev),
                                           p_out=out[:, 1], **plan)
    want_t = logits.float().argmax(-1)  # torch: first maximal column, NaN the maximum
    assert torch.equal(target.cpu(), want_t)
    want_p = pkg.batched_probabilities(ld[rows.to(dev)], t.to(dev), k.to(dev), p.to(dev), **plan)
    assert torch.equal(out[:, 1].cpu().view(torch.int32), want_p.cpu().view(torch.int32))
    assert bool((out[:, 0] == -1).all()) and bool((out[:, 2] == -1).all())


@pytest.mark.parametrize("dtype,vocab,n,w1,filtered", [
    (torch.bfloat16, 32000, 6, 4, True),
    (torch.float32, 1000, 3, 1, True),
    (torch.float16, 151936, 2, 3, True),
    (torch.bfloat16, 5000, 40, 8, True),
    (torch.float32, 49152, 32, 4, True),
    (torch.float32, 20000, 8, 3, True),  # LDS chunks past V, a partial last cascade group
    (torch.float32, 12289, 4, 32, True),  # the 32-draft limit, V off the 4-float alignment
    # no row filtered: the row-split distributions, whose write launch also sums p
    (torch.float32, 65536, 24, 4, False),
    (torch.float32, 49152, 32, 4, False),
    (torch.bfloat16, 40000 + 3, 5, 2, False),
    (torch.float16, 300, 4, 3, False),
    (torch.float32, 8191, 3, 16, False),
])
def test_verify_accept_equals_the_separate_calls(pkg, dev, dtype, vocab, n, w1, filtered):
    """verify_accept (distributions, argmax targets and the draft rows' partial sums in
    one launch, then the acceptance) is bitwise verify_distributions over every row
    followed by speculative_accept; its targets equal torch's argmax (NaN rows, ties at
    the maximum, signed zeros, all -inf rows).  The p rows' row sums are formed on chip
    for 16 register chunks (V in (16384, 49152]: 20000, 32000, 49152) and read back
    otherwise, both in one launch when a flat row takes the exact path."""
    _say("verify accept", dtype, vocab, n, w1, filtered)
    g = torch.Generator().manual_seed(vocab + n)
    rows = n * (w1 + 1)
    logits = (torch.randn(n, w1 + 1, vocab, generator=g) * 3).to(dtype)
    if not filtered:
        logits[1, 2, 7] = float("nan")  # a NaN row: NaN p, an error for its request
    else:
        # argmax targets: a NaN (the maximum), a tie at the maximum (the first column),
        # an all-zero row with -0.0 first, an all -inf row
        logits[0, 1, vocab // 2] = float("nan")
        logits[0, 1, vocab - 1] = float("nan")
        top = logits[1, 0].float().max() + 1
        logits[1, 0, vocab - 2] = top
        logits[1, 0, 3 if vocab > 3 else 0] = top
        logits[-1, -1] = 0.0
        logits[-1, -1, 0] = -0.0
        logits[-1, 0] = float("-inf")
        # a flat row: its top-p cut falls in a bin of every token (the exact path,
        # whose row sums are read back) beside rows whose sums are formed on chip
        logits[0, 0] = 1.5
    t = torch.rand(rows, generator=g) + 0.5
    k = torch.where(torch.rand(rows, generator=g) < 0.3, 40, -1)
    p = torch.where(torch.rand(rows, generator=g) < 0.5, 0.9, 1.0)
    if not filtered:
        k, p = torch.full((rows,), -1), torch.ones(rows)
    else:
        k[0], p[0] = -1, 0.9  # the flat row's top-p cut
        k[1], p[1] = 1, 1.0  # top-k 1: one kept token, from the cut bin's list
        k[2], p[2] = -1, 0.0  # top-p 0 keeps one token
    plan = _host_args(k.tolist(), p.tolist(), vocab)
    q = (torch.randn(n, w1, vocab, generator=g) * 2).softmax(-1)
    u = torch.rand(n, 2 * w1 + 1, generator=g)
    draft_tok = torch.stack([osamp.categorical(q[:, j], u[:, j])[0] for j in range(w1)], 1)
    drafts = torch.randint(0, w1 + 1, (n,), generator=g)
    args = [x.to(dev) for x in (logits, t, k, p, draft_tok, drafts, q,
                                u[:, w1:2 * w1].contiguous(), u[:, 2 * w1].contiguous())]
    target, p_o, res = pkg.verify_accept(*args, **plan)
    want_t, want_p = pkg.verify_distributions(args[0].view(rows, vocab),
                                              torch.arange(rows, device=dev), args[1], args[2],
                                              args[3], **plan)
    want = pkg.speculative_accept(args[4], args[5], args[6], want_p.view(n, w1 + 1, vocab),
                                  args[7], args[8])
    assert torch.equal(target.cpu(), want_t.cpu())
    assert torch.equal(target.cpu(), logits.view(rows, vocab).float().argmax(-1))
    assert torch.equal(p_o.cpu().view(torch.int32), want_p.view(n, w1 + 1, vocab).cpu().view(torch.int32))
    for a, b, name in zip(res, want, want._fields):
        assert torch.equal(a.cpu(), b.cpu()), name


# ------------------------------------------------------------ row-split form

def _probs_abi(dev, logits, t, k, p, plan, split, out=None):
    """rlt_batched_probabilities through the C ABI: the row-split form (workspace of the
    queried size) or the single-workgroup form (no workspace)."""
    from vllm_rlt_amd import _lib

    lib = _lib.library()
    n, vocab = logits.shape
    out = torch.full((n, vocab), -7.0, device=dev) if out is None else out
    nbytes = lib.rlt_probabilities_workspace_size(n, 0, vocab) if split else 0
    assert nbytes > 0 or not split
    ws = _lib.workspace(nbytes, dev) if split else None
    status = lib.rlt_batched_probabilities(
        _lib.ptr(logits), _lib.dtype_code(logits.dtype), logits.stride(0), n, vocab,
        _lib.ptr(t), _lib.ptr(k), _lib.ptr(p), plan["max_top_k"], int(plan["apply_top_p"]),
        _lib.ptr(out), out.stride(0), _lib.ptr(ws), nbytes, _lib.stream_of(dev))
    _lib.check(status, "rlt_batched_probabilities")
    torch.cuda.synchronize(dev)
    return out


@pytest.mark.parametrize("name,n,vocab,dtype,stride_pad", [
    ("config4-rows", 80, 65536, torch.float32, 0),    # 64 columns per thread
    ("config5-rows", 1280, 65536, torch.float32, 0),
    ("config1-q", 128, 49152, torch.float32, 0),       # 16 per thread
    ("few-rows", 8, 65536, torch.bfloat16, 0),
    ("tiny", 5, 1, torch.float32, 0),
    ("small", 7, 17, torch.float16, 0),
    ("odd-vocab", 24, 4097, torch.float32, 0),        # scalar loads (V % 4 != 0)
    ("odd-stride", 24, 3000, torch.float16, 3),       # scalar loads (row stride % 4 != 0)
    ("big-vocab", 6, 151936, torch.float32, 0),
    ("max-vocab", 3, 262144, torch.bfloat16, 0),
])
def test_split_form_matches_single_workgroup_form(pkg, dev, name, n, vocab, dtype, stride_pad):
    """Calls that filter no row run the row-split form when given a workspace: the same
    values as the single-workgroup form (their float64 totals are summed in different
    orders: 1e-6 relative), NaN rows alike, and the oracle's values."""
    _say("split vs single", name)
    g = torch.Generator().manual_seed(zlib.crc32(name.encode()))
    scale = torch.tensor([3.0, 0.5, 6.0, 1e-3, 2.0, 30.0])[torch.arange(n) % 6][:, None]
    base = torch.randn(n, vocab + stride_pad, generator=g) * scale
    logits = base.to(dtype).to(dev)[:, :vocab]
    tt = torch.tensor([0.7, 1.0, 0.5, 1.0, 1.3, 0.9])[torch.arange(n) % 6]
    tk = torch.full((n,), -1, dtype=torch.int64)
    tp = torch.ones(n)
    if n > 2:
        logits[2, vocab // 3] = float("nan")  # a NaN row
    if n > 4:
        logits[4] = -torch.inf                # no finite logit: NaN row
    plan = {"max_top_k": 0, "apply_top_p": False}
    args = [x.to(dev) for x in (tt, tk, tp)]
    a = _probs_abi(dev, logits, *args, plan, split=True).cpu()
    b = _probs_abi(dev, logits, *args, plan, split=False).cpu()
    assert torch.equal(a.isnan(), b.isnan())
    torch.testing.assert_close(a, b, atol=0, rtol=1e-6, equal_nan=True)
    # against float64 softmax(l / T) (torch's float32 total drifts past 1e-5 at these
    # widths), and against the oracle where its own total is accurate
    sel = [i for i in range(min(n, 6)) if i not in (2, 4)]
    x64 = logits[sel].double().cpu() / tt[sel].double()[:, None]
    torch.testing.assert_close(a[sel].double(), x64.softmax(-1), atol=ATOL, rtol=RTOL)
    if vocab <= 65536:
        want = osamp.batched_probabilities(logits[sel].float().cpu(), tt[sel], tk[sel], tp[sel], **plan)
        torch.testing.assert_close(a[sel], want, atol=ATOL, rtol=RTOL)
    if n > 4:
        assert torch.isnan(a[2]).all() and torch.isnan(a[4]).all()


def test_split_form_output_stride_and_filtered_calls(pkg, dev):
    """Output rows wider than V keep their columns past V; a filtering call ignores the
    workspace and runs the single-workgroup form (bitwise equal)."""
    _say("split output stride")
    g = torch.Generator().manual_seed(5)
    n, vocab = 10, 12000
    logits = (torch.randn(n, vocab, generator=g) * 3).to(dev)
    t = torch.full((n,), 0.8, device=dev)
    k = torch.full((n,), -1, dtype=torch.int64, device=dev)
    p = torch.full((n,), 0.9, device=dev)
    plan = {"max_top_k": 0, "apply_top_p": False}
    wide = torch.full((n, vocab + 5), -7.0, device=dev)
    a = _probs_abi(dev, logits, t, k, p, plan, split=True, out=wide)
    assert bool((a[:, vocab:] == -7.0).all())
    b = _probs_abi(dev, logits, t, k, p, plan, split=False)
    torch.testing.assert_close(a[:, :vocab], b, atol=0, rtol=1e-6)
    plan = {"max_top_k": 0, "apply_top_p": True}
    a = _probs_abi(dev, logits, t, k, p, plan, split=True)
    b = _probs_abi(dev, logits, t, k, p, plan, split=False)
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_split_form_is_batch_invariant(pkg, dev):
    """A row's statistics come from fixed 4096-column blocks, whatever the slice width
    (16, 32 or 64 columns per thread; verify_accept's 32 against verify_distributions' 16
    is compared bitwise in test_verify_accept_equals_the_separate_calls): a row gives the
    same bits in a batch of 1024 rows as alone."""
    _say("split batch invariance")
    g = torch.Generator().manual_seed(9)
    n, vocab = 1024, 65536
    logits = (torch.randn(n, vocab, generator=g) * 3).to(dev)
    t = torch.full((n,), 0.9, device=dev)
    k = torch.full((n,), -1, dtype=torch.int64, device=dev)
    p = torch.ones(n, device=dev)
    plan = {"max_top_k": 0, "apply_top_p": False}
    big = _probs_abi(dev, logits, t, k, p, plan, split=True)
    for rows in ([5], [0, 700, 1023]):
        idx = torch.tensor(rows, device=dev)
        small = _probs_abi(dev, logits[idx].contiguous(), t[idx], k[idx], p[idx], plan, split=True)
        assert torch.equal(small.view(torch.int32), big[idx].view(torch.int32)), rows
