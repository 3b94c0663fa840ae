"""MI355X sampling distributions and acceptance sampler behind the reference sampler API.

Same signatures, dtypes, shape errors and flag-not-raise conventions as
vllm_rlt/worker/speculative_sampling.py (``batched_probabilities`` :8-56,
``categorical`` :59-85, ``AcceptResult`` :88-101, ``speculative_accept``
:104-181), plus the device greedy round of vllm_rlt/worker/async_speculative.py:706-720
(``greedy_accept_batched``).  Acceptance and categorical results are
bit-exact with the reference formula computed by torch on the CPU when fed
identical fp32 probabilities and uniforms (the import-time guard below checks
that this host's torch sums in that order); against the formula computed by
torch on the GPU they can differ only at decisions within float32 rounding of
the masses.  Every call enqueues gfx950 kernels on the current
stream without host synchronization; inputs are never modified.
"""

import warnings
from typing import NamedTuple

import numpy as np
import torch

from . import _lib


# ------------------------------------------------------- torch-CPU sum-order guard
#
# The acceptance kernels reproduce the summation order of torch's CPU
# ``Tensor.sum(-1, dtype=float32)`` (32 streams of a 4-level cascade over 8-lane
# vectors, 4 in flight), which is what makes them bit-exact with the reference run
# on the CPU.  Another torch build or CPU dispatch (e.g. 16-lane vectors) would
# sum in another order, and the bit-exact claim would silently stop holding.  At
# import the host's torch sums order-sensitive rows and compares the bits with the
# values the kernels produce (pinned by a GPU test); a mismatch warns and is
# recorded in CPU_SUM_ORDER_MATCHES.

def order_fixture(vocab):
    """Deterministic float32 row whose float32 sum depends on the summation order
    (values spread over 2^-11 .. 2^11)."""
    i = np.arange(vocab, dtype=np.uint64)
    frac = ((i * np.uint64(2654435761)) % np.uint64(1 << 32)).astype(np.float64) / 2.0**32
    scale = np.exp2(((i * np.uint64(7)) % np.uint64(23)).astype(np.int64) - 11)
    return (frac * scale).astype(np.float32)


# float32 bits of order_fixture(V).sum() in the kernels' order, per V
ORDER_FIXTURE_SUMS = {7: 0x4484407F, 1000: 0x47AB9584, 49152: 0x4A8587B4, 65536: 0x4AB1FE4C,
                      151936: 0x4B4E6A2B}


def _host_sum_order_matches():
    for vocab, bits in ORDER_FIXTURE_SUMS.items():
        x = torch.from_numpy(order_fixture(vocab)).view(1, vocab)
        got = int(x.sum(-1, dtype=torch.float32).view(torch.int32)[0]) & 0xFFFFFFFF
        if got != bits:
            return False
    return True


CPU_SUM_ORDER_MATCHES = _host_sum_order_matches()
if not CPU_SUM_ORDER_MATCHES:
    warnings.warn(
        "this host's torch sums float32 rows in another order than the one the MI355X "
        "acceptance kernels reproduce: their results are not bit-exact with the reference "
        "run on this host's CPU (they still follow the reference's formula)", RuntimeWarning)


class AcceptResult(NamedTuple):
    """Device-side verification result; reference: speculative_sampling.py:88-101."""

    tokens: torch.Tensor
    accepted: torch.Tensor
    final: torch.Tensor
    error: torch.Tensor


def _f32(t):
    t = t if t.dtype == torch.float32 else t.float()
    return t if t.is_contiguous() else t.contiguous()


def _i64(t):
    t = t if t.dtype == torch.int64 else t.long()
    return t if t.is_contiguous() else t.contiguous()


_LOGIT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _rows(t):
    """Logits with unit column stride (row stride free), in a supported dtype."""
    if t.dtype not in _LOGIT_DTYPES:
        t = t.float()
    return t if t.stride(-1) == 1 else t.contiguous()


def _request_rows(t):
    """``[n, W1 + 1, V]`` logits whose rows are one evenly strided ``[n * (W1 + 1), V]``
    view, in a supported dtype (the layout the greedy and verify kernels read)."""
    t = _rows(t)
    return t if t.stride(0) == t.shape[1] * t.stride(1) else t.contiguous()


# The C++ operators raise on a dtype or layout they do not read; these wrappers make
# the conversions the reference's own functions make (``logits.float()``,
# ``drafts.long()``, speculative_sampling.py:39,131-146), and only when needed.


def batched_probabilities(logits, temperature, top_k, top_p, *, max_top_k, apply_top_p):
    """Temperature / strict top-k / top-p distribution of every row as ``[n, V]`` float32.

    reference: vllm_rlt/worker/speculative_sampling.py:8-56.  ``max_top_k`` and
    ``apply_top_p`` come from the host plan (no host synchronization happens here).
    Tokens tied at a top-k or top-p cut survive in column order (the reference
    leaves the surviving index of a tie unspecified).  Runs the C++ operator
    ``torch.ops.rlt_mi355x.spec_probs``.
    """
    _lib.require_gpu(logits, temperature, top_k, top_p)
    return _lib.ops().spec_probs(_rows(logits), _f32(temperature), _i64(top_k), _f32(top_p),
                                 int(max_top_k), bool(apply_top_p))


def greedy_accept_batched(draft_tokens, drafts, target_logits):
    """Device greedy round: argmax per verify row, then the leading-match count.

    reference: vllm_rlt/worker/async_speculative.py:706-720 (host rule
    vllm_rlt/worker/speculative.py:41-53).  ``target_logits`` is ``[n, W1 + 1, V]``;
    returns ``(targets int64 [n, W1 + 1], accepted int64 [n], next_token int64 [n])``
    where draft j is checked against target row j and only ``drafts[r]`` drafts count.
    Runs ``torch.ops.rlt_mi355x.greedy_accept``.
    """
    _lib.require_gpu(draft_tokens, drafts, target_logits)
    if target_logits.ndim != 3:
        raise ValueError("target_logits must be [n, W1 + 1, V]")
    return _lib.ops().greedy_accept(_i64(draft_tokens), _i64(drafts), _request_rows(target_logits))


def propose_drafts(logits, random_rows, temperature, top_k, top_p, u, *, max_top_k, apply_top_p,
                   q_out=None):
    """Draft proposals of one draft offset: ``(proposed int64 [m], q_o float32 [r, V])``.

    reference: vllm_rlt/worker/async_speculative.py:645-663 -- ``proposed =
    logits.argmax(-1)``; for the random rows ``q_o = batched_probabilities(
    logits[random_rows], temperature, top_k, top_p)``, ``proposed[random_rows] =
    categorical(q_o, u)[0]``.  ``temperature`` / ``top_k`` / ``top_p`` / ``u`` are per
    random row.  ``q_out`` (optional) is a ``[r, V]`` float32 view with unit column
    stride to write q_o into (e.g. ``q[ranks, offset]`` when ranks are contiguous:
    ``q[:, offset]``); otherwise a new tensor.
    """
    if logits.ndim != 2:
        raise ValueError("logits must be a 2-D [m, V] tensor")
    m, vocab = logits.shape
    if random_rows is None:
        random_rows = torch.empty(0, dtype=torch.int64, device=logits.device)
    if random_rows.ndim != 1:
        raise ValueError("random_rows must be 1-D")
    r = random_rows.shape[0]
    for name, value in (("temperature", temperature), ("top_k", top_k), ("top_p", top_p),
                        ("u", u)):
        if r and value.shape != (r,):
            raise ValueError(f"{name} must have shape [{r}], got {tuple(value.shape)}")
    if max_top_k < 0:
        raise ValueError("max_top_k must be nonnegative")
    _lib.require_gpu(logits, random_rows, *((temperature, top_k, top_p, u) if r else ()), q_out)
    device = logits.device
    proposed = torch.empty(m, dtype=torch.int64, device=device)
    if q_out is None:
        q_out = torch.empty((r, vocab), dtype=torch.float32, device=device)
    elif q_out.shape != (r, vocab) or q_out.dtype != torch.float32 or q_out.stride(-1) != 1:
        raise ValueError("q_out must be a float32 [r, V] view with unit column stride")
    if m == 0 and r == 0:
        return proposed, q_out
    if vocab == 0:
        raise ValueError("logits must have V >= 1")
    x = logits if logits.dtype in _LOGIT_DTYPES else logits.float()
    x = _rows(x)
    rows = _i64(random_rows)
    lib = _lib.library()
    ws = _lib.workspace(lib.rlt_propose_drafts_workspace_size(m, r, vocab), device)
    args = (_f32(temperature), _i64(top_k), _f32(top_p), _f32(u)) if r else (None,) * 4
    status = lib.rlt_propose_drafts(
        _lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), m, vocab, _lib.ptr(rows), r,
        *(_lib.ptr(a) for a in args[:3]), int(max_top_k), int(bool(apply_top_p)),
        _lib.ptr(args[3]), _lib.ptr(q_out), q_out.stride(0) if r else vocab, _lib.ptr(proposed),
        _lib.ptr(ws), ws.numel(), _lib.stream_of(device))
    _lib.check(status, "rlt_propose_drafts")
    return proposed, q_out


def verify_distributions(logits, random_rows, temperature, top_k, top_p, *, max_top_k,
                         apply_top_p, p_out=None):
    """The verify side of a round: ``(target int64 [m], p float32 [r, V])``.

    reference: vllm_rlt/worker/async_speculative.py:678-692 -- ``target =
    logits.argmax(-1)`` over every verify row, and the distributions of the random
    rows (``_probabilities(logits[v_rows], ...)``; ``temperature`` / ``top_k`` /
    ``top_p`` per random row), read straight from ``logits`` through ``random_rows``.
    ``p_out`` (optional): a ``[r, V]`` float32 view with unit column stride.
    """
    if logits.ndim != 2:
        raise ValueError("logits must be a 2-D [m, V] tensor")
    m, vocab = logits.shape
    if random_rows is None:
        random_rows = torch.empty(0, dtype=torch.int64, device=logits.device)
    if random_rows.ndim != 1:
        raise ValueError("random_rows must be 1-D")
    r = random_rows.shape[0]
    for name, value in (("temperature", temperature), ("top_k", top_k), ("top_p", top_p)):
        if r and value.shape != (r,):
            raise ValueError(f"{name} must have shape [{r}], got {tuple(value.shape)}")
    if max_top_k < 0:
        raise ValueError("max_top_k must be nonnegative")
    _lib.require_gpu(logits, random_rows, *((temperature, top_k, top_p) if r else ()), p_out)
    if p_out is None and r:
        # new output rows: the C++ operator torch.ops.rlt_mi355x.verify_distributions
        return tuple(_lib.ops().verify_distributions(
            _rows(logits), _i64(random_rows), _f32(temperature), _i64(top_k), _f32(top_p),
            int(max_top_k), bool(apply_top_p)))
    device = logits.device
    target = torch.empty(m, dtype=torch.int64, device=device)
    if p_out is None:
        p_out = torch.empty((r, vocab), dtype=torch.float32, device=device)
    elif p_out.shape != (r, vocab) or p_out.dtype != torch.float32 or p_out.stride(-1) != 1:
        raise ValueError("p_out must be a float32 [r, V] view with unit column stride")
    if m == 0 and r == 0:
        return target, p_out
    if vocab == 0:
        raise ValueError("logits must have V >= 1")
    x = logits if logits.dtype in _LOGIT_DTYPES else logits.float()
    x = _rows(x)
    args = (_f32(temperature), _i64(top_k), _f32(top_p)) if r else (None,) * 3
    lib = _lib.library()
    nbytes = lib.rlt_probabilities_workspace_size(r, m, vocab) if r else 0
    ws = _lib.workspace(nbytes, device) if nbytes else None
    status = lib.rlt_verify_distributions(
        _lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), m, vocab, _lib.ptr(_i64(random_rows)),
        r, *(_lib.ptr(a) for a in args), int(max_top_k), int(bool(apply_top_p)), _lib.ptr(p_out),
        p_out.stride(0) if r else vocab, _lib.ptr(target), _lib.ptr(ws), nbytes,
        _lib.stream_of(device))
    _lib.check(status, "rlt_verify_distributions")
    return target, p_out


def categorical(weights, u):
    """Inverse-CDF draw from ``[m, V]`` nonnegative weights with ``[m]`` uniforms.

    Returns ``(index int64 [m], valid bool [m])``; reference: speculative_sampling.py:59-85.
    Runs ``torch.ops.rlt_mi355x.categorical``.
    """
    _lib.require_gpu(weights, u)
    return _lib.ops().categorical(_f32(weights), _f32(u))


def speculative_accept(draft_tokens, drafts, q, p, u_accept, u_final):
    """Batched speculative rejection sampling; reference: speculative_sampling.py:104-181.
    Runs ``torch.ops.rlt_mi355x.spec_accept``."""
    _lib.require_gpu(draft_tokens, drafts, q, p, u_accept, u_final)
    return AcceptResult(*_lib.ops().spec_accept(_i64(draft_tokens), _i64(drafts), _f32(q), _f32(p),
                                                _f32(u_accept), _f32(u_final)))


def verify_accept(target_logits, temperature, top_k, top_p, draft_tokens, drafts, q, u_accept,
                  u_final, *, max_top_k, apply_top_p):
    """The stochastic verify round in one call: ``(target, p, AcceptResult)``.

    ``target, p = verify_distributions(target_logits.view(-1, V), all rows, ...)`` and
    ``speculative_accept(draft_tokens, drafts, q, p.view(n, W1 + 1, V), u_accept,
    u_final)``, bitwise (reference: vllm_rlt/worker/async_speculative.py:678-692 then
    :727-734).  The draft rows' row sums are computed by otherwise idle workgroups of
    the distribution launch.  ``temperature`` / ``top_k`` / ``top_p`` are per verify row
    ``[n * (W1 + 1)]``; ``target`` is ``[n * (W1 + 1)]``.  Runs
    ``torch.ops.rlt_mi355x.verify_accept``.
    """
    _lib.require_gpu(target_logits, temperature, top_k, top_p, draft_tokens, drafts, q, u_accept,
                     u_final)
    if target_logits.ndim != 3:
        raise ValueError("target_logits must be [n, W1 + 1, V]")
    out = _lib.ops().verify_accept(_request_rows(target_logits), _f32(temperature), _i64(top_k),
                                   _f32(top_p), _i64(draft_tokens), _i64(drafts), _f32(q),
                                   _f32(u_accept), _f32(u_final), int(max_top_k),
                                   bool(apply_top_p))
    return out[0], out[1], AcceptResult(*out[2:])


# ------------------------------------------------------------ sync-mode rejection

REJECT_ALL_ACCEPTED, REJECT_REJECTED, REJECT_ZERO_MASS, REJECT_BAD_RESIDUAL, REJECT_BAD_TOKEN = range(5)


def rejection_rows(candidates, counts, target, proposal, uniforms, *, sum_threads=1):
    """Device part of sync-mode rejection sampling for a batch: ``(status int32 [n],
    accepted int64 [n], residual float32 [n, V])``.

    reference: vllm_rlt/worker/speculative.py:56-72 (``rejection_sample``) as
    ``_collect_round`` (:574-625) applies it draft after draft.  ``candidates`` int64
    ``[n, K]``, ``counts`` ``[n]`` (drafts per request), ``target`` float32
    ``[n, K + 1, V]``, ``proposal`` ``[n, K, V]``, ``uniforms`` ``[n, K]``.  Status:
    0 all drafts accepted, 1 rejected at ``accepted`` (``residual`` row = the normalized
    residual), 2 zero proposal mass, 3 invalid residual mass, 4 candidate out of range.
    The residual total follows one fixed summation order, whatever the calling process's
    thread count: torch's CPU order for ``residual.sum()`` on ``sum_threads`` threads
    (default 1, the single-thread order; pass the thread count of a CPU run to reproduce
    that run bit for bit).  Against the reference run on device tensors, whose total is
    torch-ROCm's reduction, the total may differ by a few float32 ulps; only a
    multinomial draw that lands that close to a CDF boundary can then differ.
    """
    if candidates.ndim != 2:
        raise ValueError("candidates must be [n, K]")
    n, k = candidates.shape
    if target.ndim != 3 or target.shape[:2] != (n, k + 1):
        raise ValueError("target must be [n, K + 1, V]")
    vocab = target.shape[-1]
    if proposal.shape != (n, k, vocab) or uniforms.shape != (n, k) or counts.shape != (n,):
        raise ValueError("proposal must be [n, K, V], uniforms [n, K] and counts [n]")
    return _launch_rejection(candidates, counts, target, proposal, uniforms, k, sum_threads)


def _launch_rejection(candidates, counts, target, proposal, uniforms, k, sum_threads):
    """rlt_rejection_sample on rows whose layout the caller has checked (target rows
    j > count of a request are never read, so one verified draft may pass a [1, 1, V]
    target)."""
    n, vocab = candidates.shape[0], target.shape[-1]
    threads = int(sum_threads)
    if threads < 1:
        raise ValueError("sum_threads must be a positive thread count")
    _lib.require_gpu(candidates, counts, target, proposal, uniforms)
    device = target.device
    status = torch.empty(n, dtype=torch.int32, device=device)
    accepted = torch.empty(n, dtype=torch.int64, device=device)
    residual = torch.empty((n, vocab), dtype=torch.float32, device=device)
    if n == 0:
        return status, accepted, residual
    lib = _lib.library()
    ws = _lib.workspace(lib.rlt_rejection_sample_workspace_size(n, vocab, threads), device)
    st = lib.rlt_rejection_sample(
        _lib.ptr(_i64(candidates)), _lib.ptr(_i64(counts)), _lib.ptr(_f32(target)),
        _lib.ptr(_f32(proposal)), _lib.ptr(_f32(uniforms)), n, k, vocab, threads,
        _lib.ptr(status), _lib.ptr(accepted), _lib.ptr(residual), _lib.ptr(ws), ws.numel(),
        _lib.stream_of(device))
    _lib.check(st, "rlt_rejection_sample")
    return status, accepted, residual


def _raise_for(status, what=""):
    if status == REJECT_ZERO_MASS:
        raise ValueError("candidate has zero proposal probability" + what)
    if status == REJECT_BAD_TOKEN:
        raise IndexError("candidate is outside the vocabulary" + what)
    if status == REJECT_BAD_RESIDUAL:
        raise RuntimeError("invalid speculative residual probability mass" + what)


def rejection_sample(candidate, target, proposal, generator):
    """Return ``(token, accepted)`` for one draft; reference:
    vllm_rlt/worker/speculative.py:56-72.

    ``target`` / ``proposal`` are the normalized float32 ``[V]`` rows of p and q on the
    device, ``generator`` the request's generator on that device.  The generator is
    consumed exactly as the reference consumes it: one ``torch.rand(())`` unless the
    candidate has no proposal mass, then one ``torch.multinomial`` draw on a rejection.
    One host read of the outcome instead of the reference's three to four.
    """
    device = target.device
    vocab = target.shape[-1]
    if target.shape != (vocab,) or proposal.shape != (vocab,):
        raise ValueError("target and proposal must be [V] rows")
    before = generator.get_state()
    u = torch.rand((), device=device, generator=generator)
    cand = torch.tensor([[int(candidate)]], dtype=torch.int64).to(device, non_blocking=True)
    counts = torch.ones(1, dtype=torch.int64, device=device)
    # one draft: row 0 of the target is all the kernel reads
    status, _, residual = _launch_rejection(cand, counts, target.view(1, 1, vocab),
                                            proposal.view(1, 1, vocab), u.view(1, 1), 1, 1)
    code = int(status[0])
    if code in (REJECT_ZERO_MASS, REJECT_BAD_TOKEN):
        generator.set_state(before)  # the reference raises before drawing u
    _raise_for(code)
    if code == REJECT_ALL_ACCEPTED:
        return candidate, True
    return int(torch.multinomial(residual[0], 1, generator=generator).squeeze(0).item()), False


def rejection_round(candidates, target, proposal, generators, *, sum_threads=1):
    """The stochastic branch of the synchronous runner's round for a batch of requests:
    a list of ``(tokens, accepted)`` per request.

    reference: vllm_rlt/worker/speculative.py:574-625 (``_collect_round``, requests with
    temperature > 0).  ``candidates[i]``: request i's draft ids (host ints, at most K);
    ``target`` float32 ``[n, K + 1, V]``: p of each verify row (row ``len(candidates[i])``
    is the bonus row); ``proposal`` ``[n, K, V]``: the draft distributions q;
    ``generators[i]``: request i's generator on the device.  Every generator ends in the
    state the reference leaves it in and every token equals the reference's given the
    same p and q rows: each request's uniforms are drawn in the reference's order before
    one batched launch decides every request, and the generator is then rewound to just
    after the uniforms the reference would have drawn before its residual or bonus
    ``torch.multinomial``.  Errors are raised as the reference raises them, for the
    first failing request, with the generators of later requests untouched.  Requests
    must have distinct generators (a shared one is handled one request at a time).
    """
    n = len(candidates)
    if len(generators) != n or target.shape[0] != n or proposal.shape[0] != n:
        raise ValueError("candidates, target, proposal and generators must cover n requests")
    if len({id(g) for g in generators}) != n:
        return [rejection_round([candidates[i]], target[i:i + 1], proposal[i:i + 1],
                                [generators[i]], sum_threads=sum_threads)[0] for i in range(n)]
    k = proposal.shape[1]
    device = target.device
    counts = [len(c) for c in candidates]
    if any(c > k for c in counts):
        raise ValueError("a request has more candidates than proposal rows")
    states, uniforms = [], []
    for gen, d in zip(generators, counts):
        st = [gen.get_state()]
        row = []
        for _ in range(d):
            row.append(torch.rand((), device=device, generator=gen))
            st.append(gen.get_state())
        row += [torch.zeros((), device=device)] * (k - d)
        uniforms.append(torch.stack(row) if row else torch.zeros(0, device=device))
        states.append(st)
    u = torch.stack(uniforms) if n else torch.zeros((0, k), device=device)
    cand = torch.tensor([c + [0] * (k - len(c)) for c in candidates], dtype=torch.int64)
    cand = cand.view(n, k).to(device, non_blocking=True)
    cnt = torch.tensor(counts, dtype=torch.int64).to(device, non_blocking=True)
    status, accepted, residual = rejection_rows(cand, cnt, target, proposal, u,
                                                sum_threads=sum_threads)
    outcome = torch.stack((status.long(), accepted)).tolist()  # the one host read
    draws = []
    for i, gen in enumerate(generators):
        code, a = outcome[0][i], outcome[1][i]
        if code != REJECT_ALL_ACCEPTED and code != REJECT_REJECTED:
            consumed = a + 1 if code == REJECT_BAD_RESIDUAL else a
            gen.set_state(states[i][consumed])
            for j in range(i + 1, n):
                generators[j].set_state(states[j][0])
            _raise_for(code, f" (request {i}, draft {a})")
        if code == REJECT_REJECTED:
            gen.set_state(states[i][a + 1])
            draws.append(torch.multinomial(residual[i], 1, generator=gen))
        else:
            draws.append(torch.multinomial(target[i, counts[i]], 1, generator=gen))
    drawn = torch.cat(draws).tolist() if draws else []
    results = []
    for i in range(n):
        a = outcome[1][i]
        results.append((list(candidates[i][:a]) + [int(drawn[i])], a))
    return results


def row_mass(x):
    """``x.sum(-1, dtype=float32)`` of a 2-D fp32 tensor in torch-CPU summation order."""
    if x.ndim != 2:
        raise ValueError("x must be 2-D")
    _lib.require_gpu(x)
    rows, vocab = x.shape
    out = torch.empty(rows, dtype=torch.float32, device=x.device)
    if rows == 0:
        return out
    xx = _f32(x)
    lib = _lib.library()
    ws = _lib.workspace(lib.rlt_row_mass_workspace_size(rows, vocab), x.device)
    status = lib.rlt_row_mass_f32(_lib.ptr(xx), rows, vocab, _lib.ptr(out), _lib.ptr(ws),
                                  ws.numel(), _lib.stream_of(x.device))
    _lib.check(status, "rlt_row_mass_f32")
    return out


def greedy_accept(candidates, targets):
    """Host prefix match of one request; reference: vllm_rlt/worker/speculative.py:41-53.

    ``targets[j]`` is the target argmax of verify row j.  Returns the committed
    tokens (the target prefix through the first mismatch) and the accepted count.
    """
    accepted = 0
    for candidate, target in zip(candidates, targets):
        if candidate != target:
            break
        accepted += 1
    return list(targets[: accepted + 1]), accepted


class RandomRoundMerge(NamedTuple):
    """reference: vllm_rlt/worker/async_speculative.py:152-159."""

    rows: torch.Tensor  # [R] result rows (committed sequences for random requests)
    accepted: torch.Tensor  # [n]
    next_tokens: torch.Tensor  # [n]
    next_positions: torch.Tensor  # [n] starts + accepted + 1
    next_values: torch.Tensor  # [n, 2] (token, position) to scatter into the slot table
    error: torch.Tensor  # [n] int64 0/1 flags


def merge_random_round(target, accepted, next_tokens, starts, input_tokens, result,
                       random_requests, verify_rows, verify_ranks, verify_offsets):
    """Overlay the random requests' outcome on the greedy round in one launch, no host reads.

    reference: vllm_rlt/worker/async_speculative.py:162-198.  ``random_requests`` and the
    ``verify_*`` index arrays may be device tensors or host arrays (copied to the device);
    an index must not repeat.  An index outside its range (where the reference's
    indexing raises) is skipped and fails the whole round: ``error`` is 1 for every
    request, and every request keeps its ``(input_token, start)`` slot values.
    """
    device = target.device
    _lib.require_gpu(target, accepted, next_tokens, starts, input_tokens, *result)

    def idx(x):
        return _i64(torch.as_tensor(x, dtype=torch.int64, device=device))

    req, vrow, vrank, voff = (idx(x) for x in (random_requests, verify_rows, verify_ranks,
                                               verify_offsets))
    n, num_rows = starts.shape[0], target.shape[0]
    if accepted.shape != (n,) or next_tokens.shape != (n,) or input_tokens.shape != (n,):
        raise ValueError("accepted, next_tokens, starts and input_tokens must be [n]")
    r = req.shape[0]
    tokens = _i64(result.tokens)
    if tokens.dim() != 2 or tokens.shape[0] != r or result.accepted.shape != (r,) \
            or result.final.shape != (r,) or result.error.shape != (r,):
        raise ValueError("result must hold one row per random request")
    if not (vrow.shape == vrank.shape == voff.shape) or vrow.dim() != 1:
        raise ValueError("verify_rows, verify_ranks and verify_offsets must be equal-length 1-D")
    err_in = result.error if result.error.dtype == torch.bool else result.error != 0
    err_in = err_in.contiguous()
    rows = torch.empty(num_rows, dtype=torch.int64, device=device)
    acc = torch.empty(n, dtype=torch.int64, device=device)
    nxt = torch.empty(n, dtype=torch.int64, device=device)
    pos = torch.empty(n, dtype=torch.int64, device=device)
    values = torch.empty((n, 2), dtype=torch.int64, device=device)
    error = torch.empty(n, dtype=torch.int64, device=device)
    tg, ac, nt, st, it = (_i64(x) for x in (target, accepted, next_tokens, starts, input_tokens))
    ra, rf = _i64(result.accepted), _i64(result.final)
    lib = _lib.library()
    status = lib.rlt_merge_random_round(
        _lib.ptr(tg), num_rows, _lib.ptr(ac), _lib.ptr(nt), _lib.ptr(st), _lib.ptr(it), n,
        _lib.ptr(tokens), tokens.shape[1], _lib.ptr(ra), _lib.ptr(rf), _lib.ptr(err_in),
        _lib.ptr(req), r, _lib.ptr(vrow), _lib.ptr(vrank), _lib.ptr(voff), vrow.shape[0],
        _lib.ptr(rows), _lib.ptr(acc), _lib.ptr(nxt), _lib.ptr(pos), _lib.ptr(values),
        _lib.ptr(error), _lib.stream_of(device))
    _lib.check(status, "rlt_merge_random_round")
    return RandomRoundMerge(rows, acc, nxt, pos, values, error)
