"""Torch-CPU restatement of the reference acceptance sampler (test oracle only).

The bit-exact acceptance contract is defined by torch-CPU arithmetic: the fp32
row sums of ``Tensor.sum(-1, dtype=float32)``, fp32 division and comparison,
and the sequential float64 ``cumsum`` + ``searchsorted(right=True)`` of the
inverse-CDF draw.  This module therefore calls the same torch ops in the same
order as the reference.  ``oracle/order.c`` models those two summation orders
independently, and the tests pin that model against torch bit for bit.
"""

from typing import NamedTuple

import numpy as np
import torch


def sampler_probabilities(logits, temperature, top_k, top_p):
    """One row's temperature / strict top-k / top-p distribution.

    reference: vllm_rlt/worker/sampler.py:28-55.
    """
    if temperature == 0:
        raise ValueError("greedy decoding has no temperature-scaled distribution")
    x = logits.float() / temperature
    if top_k > 0:
        vals, idx = x.topk(min(top_k, x.numel()))
        x = torch.full_like(x, -torch.inf).scatter_(0, idx, vals)
    if top_p < 1:
        sx, idx = x.sort(descending=True)
        drop = sx.softmax(-1).cumsum(-1) > top_p
        drop[1:] = drop[:-1].clone()
        drop[0] = False
        x = x.scatter(0, idx, sx.masked_fill(drop, -torch.inf))
    return x.softmax(-1)


def batched_probabilities(logits, temperature, top_k, top_p, *, max_top_k, apply_top_p):
    """Batched form; reference: vllm_rlt/worker/speculative_sampling.py:8-56."""
    if logits.ndim != 2:
        raise ValueError("logits must be a 2-D [n, V] tensor")
    n, vocab = logits.shape
    for name, t in (("temperature", temperature), ("top_k", top_k), ("top_p", top_p)):
        if t.shape != (n,):
            raise ValueError(f"{name} must have shape [{n}], got {tuple(t.shape)}")
    if max_top_k < 0:
        raise ValueError("max_top_k must be nonnegative")
    x = logits.float() / temperature.float()[:, None]
    if max_top_k > 0:
        k_eff = torch.where((top_k > 0) & (top_k < vocab), top_k, vocab)
        vals, idx = x.topk(min(max_top_k, vocab), dim=-1)
        keep = torch.arange(vals.shape[-1]) < k_eff[:, None]
        trimmed = torch.full_like(x, -torch.inf).scatter_(1, idx, vals.masked_fill(~keep, -torch.inf))
        x = torch.where((k_eff < vocab)[:, None], trimmed, x)
    if apply_top_p:
        tp = top_p.float()[:, None]
        sx, idx = x.sort(dim=-1, descending=True)
        drop = (sx.softmax(-1).cumsum(-1) > tp) & (tp < 1)
        drop[:, 1:] = drop[:, :-1].clone()
        drop[:, 0] = False
        x = x.scatter(1, idx, sx.masked_fill(drop, -torch.inf))
    return x.softmax(-1)


def categorical(weights, u):
    """Inverse-CDF draw; reference: vllm_rlt/worker/speculative_sampling.py:59-85."""
    if weights.ndim != 2 or weights.shape[-1] < 1:
        raise ValueError("weights must be a 2-D [m, V] tensor with V >= 1")
    if u.shape != weights.shape[:1]:
        raise ValueError(f"u must have shape [{weights.shape[0]}], got {tuple(u.shape)}")
    vocab = weights.shape[-1]
    cdf = weights.double().cumsum(-1)
    mass = cdf[:, -1]
    valid = torch.isfinite(mass) & (mass > 0)
    t = torch.minimum(u.double() * mass, torch.nextafter(mass, torch.zeros_like(mass)))
    idx = torch.searchsorted(cdf, t[:, None], right=True).squeeze(-1)
    idx = torch.where(valid, idx, torch.zeros_like(idx)).clamp(0, vocab - 1)
    return idx, valid


class AcceptResult(NamedTuple):
    tokens: torch.Tensor
    accepted: torch.Tensor
    final: torch.Tensor
    error: torch.Tensor


def speculative_accept(draft_tokens, drafts, q, p, u_accept, u_final):
    """Batched rejection sampling; reference: speculative_sampling.py:104-181."""
    n, w1 = draft_tokens.shape
    vocab = p.shape[-1]
    if drafts.shape != (n,) or u_final.shape != (n,) or u_accept.shape != (n, w1):
        raise ValueError("drafts, u_accept and u_final must match draft_tokens [n, W1]")
    if q.shape != (n, w1, vocab) or p.shape != (n, w1 + 1, vocab):
        raise ValueError("q must be [n, W1, V] and p must be [n, W1 + 1, V]")
    rows = torch.arange(n, device=p.device)
    pos = torch.arange(w1 + 1, device=p.device)
    p_mass = p.sum(-1, dtype=torch.float32)
    p_ok = torch.isfinite(p_mass) & (p_mass > 0)
    d = drafts.clamp(0, w1)
    error = drafts != d
    x = draft_tokens.clamp(0, vocab - 1)
    if w1 > 0:
        in_range = (draft_tokens >= 0) & (draft_tokens < vocab)
        q_mass = q.sum(-1, dtype=torch.float32)
        q_ok = torch.isfinite(q_mass) & (q_mass > 0)
        px = p[:, :w1].gather(2, x[..., None]).squeeze(-1).float() / p_mass[:, :w1]
        qx = q.gather(2, x[..., None]).squeeze(-1).float() / q_mass
        invalid = ~(p_ok[:, :w1] & q_ok & in_range & torch.isfinite(px) & torch.isfinite(qx) & (qx > 0))
        accept = ~invalid & ((px >= qx) | (u_accept.float() * qx < px))
        accept &= pos[None, :w1] < d[:, None]
        s = accept.long().cumprod(1).sum(1)
        at_end = s == d
        s_q = s.clamp(max=w1 - 1)
        invalid_at_s = invalid[rows, s_q] & ~at_end
        p_row = p[rows, s].float() / p_mass[rows, s][:, None]
        q_row = q[rows, s_q].float() / q_mass[rows, s_q][:, None]
        weights = torch.where(at_end[:, None], p_row, (p_row - q_row).clamp_min(0))
        stop_ok = torch.where(at_end, p_ok[rows, s], ~invalid_at_s)
    else:
        s = torch.zeros_like(d)
        weights = p[:, 0].float() / p_mass[:, :1]
        stop_ok = p_ok[:, 0]
    final, final_valid = categorical(weights, u_final)
    error = error | ~(stop_ok & final_valid)
    final = torch.where(error, torch.zeros_like(final), final)
    padded = torch.nn.functional.pad(x, (0, 1))
    tokens = torch.where(pos[None] < s[:, None], padded,
                         torch.where(pos[None] == s[:, None], final[:, None], torch.zeros_like(padded)))
    return AcceptResult(tokens, s, final, error)


def greedy_accept(candidates, targets):
    """Host form; reference: vllm_rlt/worker/speculative.py:41-53."""
    accepted = 0
    for c, t in zip(candidates, targets):
        if c != t:
            break
        accepted += 1
    return list(targets[: accepted + 1]), accepted


def greedy_accept_batched(draft_tokens, drafts, target_logits):
    """Device form of the greedy round: argmax per verify row, prefix match.

    reference: vllm_rlt/worker/async_speculative.py:706-720 (targets = argmax of
    each request-major verify row; candidate j is checked against row j).
    ``target_logits`` is [n, W1 + 1, V]; returns (targets [n, W1+1], accepted [n],
    next_token [n]).
    """
    n, w1 = draft_tokens.shape
    targets = target_logits.argmax(-1)
    live = torch.arange(w1)[None, :] < drafts[:, None]
    matches = (draft_tokens == targets[:, :w1]) & live
    accepted = matches.long().cumprod(1).sum(1)
    next_token = targets.gather(1, accepted[:, None]).squeeze(1)
    return targets, accepted, next_token


def request_uniforms(seeds, num_speculative_tokens):
    """Per-request ``torch.rand(2K + 1)`` from a fresh seeded CPU generator.

    reference: vllm_rlt/worker/async_speculative.py:567-586 (columns [0:K]
    draft draws, [K:2K] acceptance, [2K] the final draw).
    """
    rows = []
    for seed in seeds:
        g = torch.Generator().manual_seed(int(seed))
        rows.append(torch.rand((2 * num_speculative_tokens + 1,), generator=g, dtype=torch.float32))
    return torch.stack(rows)


def merge_random_round(target, accepted, next_tokens, starts, input_tokens, result,
                       random_requests, verify_rows, verify_ranks, verify_offsets):
    """Plain-Python loop restatement; reference: async_speculative.py:162-198."""
    rows = target.tolist()
    acc = accepted.tolist()
    nxt = next_tokens.tolist()
    toks = result.tokens.tolist()
    for r, rank, off in zip(verify_rows.tolist(), verify_ranks.tolist(), verify_offsets.tolist()):
        rows[r] = toks[rank][off]
    failed = [False] * len(starts)
    for rank, req in enumerate(random_requests.tolist()):
        acc[req] = int(result.accepted[rank])
        nxt[req] = int(result.final[rank])
        failed[req] = bool(result.error[rank])
    st = starts.tolist()
    inp = input_tokens.tolist()
    positions = [st[i] + acc[i] + 1 for i in range(len(st))]
    values = [[inp[i], st[i]] if failed[i] else [nxt[i], positions[i]] for i in range(len(st))]
    return (torch.tensor(rows), torch.tensor(acc), torch.tensor(nxt), torch.tensor(positions),
            torch.tensor(values), torch.tensor([int(f) for f in failed], dtype=torch.int64))


def plan_random_rows(temperatures, token_counts, num_speculative_tokens):
    """Verify-row bookkeeping of a block round's random requests (numpy).

    reference: vllm_rlt/worker/async_speculative.py:101-150 (request-major
    verify rows; draft j of a request checked against its verify row j).
    """
    counts = np.asarray(token_counts, dtype=np.int64)
    is_random = np.asarray(temperatures, dtype=np.float64) != 0
    if not is_random.any():
        return None
    requests = np.flatnonzero(is_random)
    rc = counts[requests]
    if int(rc.max()) - 1 > num_speculative_tokens:
        raise ValueError("random request has more drafts than num_speculative_tokens")
    starts = np.cumsum(counts) - counts
    verify_rows = np.concatenate([starts[i] + np.arange(counts[i]) for i in requests])
    verify_ranks = np.repeat(np.arange(len(requests)), rc)
    verify_offsets = np.concatenate([np.arange(c) for c in rc])
    return requests, verify_rows, verify_ranks, verify_offsets


def rejection_sample(candidate, target, proposal, generator):
    """One draft of the synchronous runner, on whatever device the rows live.

    reference: vllm_rlt/worker/speculative.py:56-72 (Sampler.draw:
    vllm_rlt/worker/sampler.py:57-60).
    """
    mass = proposal[candidate]
    if not bool(mass > 0):
        raise ValueError("candidate has zero proposal probability")
    uniform = torch.rand((), device=target.device, generator=generator)
    if bool(uniform * mass < target[candidate]):
        return candidate, True
    residual = (target - proposal).clamp_min(0)
    total = residual.sum()
    if not bool(torch.isfinite(total) & (total > 0)):
        raise RuntimeError("invalid speculative residual probability mass")
    return int(torch.multinomial(residual / total, 1, generator=generator).squeeze(0).item()), False


def rejection_step(candidate, target, proposal, uniform):
    """The same decision with the uniform given: ``(accepted, normalized residual or None)``.

    Raises as the reference raises.  CPU float32 rows; the residual total is torch's
    ``residual.sum()`` on this process's threads.
    """
    mass = proposal[candidate]
    if not bool(mass > 0):
        raise ValueError("candidate has zero proposal probability")
    if bool(uniform * mass < target[candidate]):
        return True, None
    residual = (target - proposal).clamp_min(0)
    total = residual.sum()
    if not bool(torch.isfinite(total) & (total > 0)):
        raise RuntimeError("invalid speculative residual probability mass")
    return False, residual / total


def collect_stochastic(candidates, target, proposal, generators):
    """The random-request branch of the synchronous round, request by request.

    reference: vllm_rlt/worker/speculative.py:601-624 (``_collect_round``); ``target[i]``
    holds request i's verify-row distributions (row ``len(candidates[i])`` is the bonus
    row), ``proposal[i]`` its draft distributions.
    """
    results = []
    for i, cands in enumerate(candidates):
        tokens, accepted = [], 0
        for offset, cand in enumerate(cands):
            token, ok = rejection_sample(cand, target[i, offset], proposal[i, offset], generators[i])
            tokens.append(token)
            if not ok:
                break
            accepted += 1
        else:
            tokens.append(int(torch.multinomial(target[i, len(cands)], 1,
                                                generator=generators[i]).squeeze(0).item()))
        results.append((tokens, accepted))
    return results
