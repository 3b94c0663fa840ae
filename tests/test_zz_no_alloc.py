"""The allocation-free acceptance entry point through the C ABI: its outputs equal
rlt_speculative_accept's (bit for bit) on two calls in a row, the second smaller,
so the shared device array's leftover contents cannot leak into a result."""

import sys

import pytest
import torch

from oracle import sampling as osamp

pytestmark = pytest.mark.gpu


def _say(*args):
    print("[case]", *args, flush=True)
    sys.stdout.flush()


def _inputs(n, w1, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    dl = torch.randn(n, w1 + 1, vocab, generator=g) * 3
    tl = dl + torch.randn(n, w1 + 1, vocab, generator=g)
    q = dl[:, :w1].softmax(-1)
    p = tl.softmax(-1)
    u = torch.rand(n, 2 * w1 + 1, generator=g)
    draft = torch.stack([osamp.categorical(q[:, j], u[:, j])[0] for j in range(w1)], 1)
    drafts = torch.randint(0, w1 + 1, (n,), generator=g)
    drafts[0] = w1
    return draft, drafts, q, p, u[:, w1:2 * w1].contiguous(), u[:, 2 * w1].contiguous()


def _call(lib, _lib, name, args, n, w1, vocab, dev, with_workspace):
    tokens = torch.full((n, w1 + 1), -7, dtype=torch.int64, device=dev)
    accepted = torch.full((n,), -7, dtype=torch.int64, device=dev)
    final = torch.full((n,), -7, dtype=torch.int64, device=dev)
    error = torch.full((n,), 7, dtype=torch.uint8, device=dev)
    outs = (tokens, accepted, final, error)
    ptrs = [_lib.ptr(a) for a in args] + [n, w1, vocab] + [_lib.ptr(o) for o in outs]
    if with_workspace:
        ws = _lib.workspace(lib.rlt_speculative_accept_workspace_size(n, w1, vocab), dev)
        st = getattr(lib, name)(*ptrs, _lib.ptr(ws), ws.numel(), _lib.stream_of(dev))
    else:
        st = getattr(lib, name)(*ptrs, _lib.stream_of(dev))
    assert st == 0, f"{name} status {st}"
    torch.cuda.synchronize(dev)
    return [o.cpu() for o in outs]


def test_noalloc_accept_matches_workspace_form_on_two_calls(pkg, dev):
    from vllm_rlt_amd import _lib

    lib = _lib.library()
    for n, w1, vocab, seed in ((32, 4, 49152, 1), (5, 3, 4099, 2)):
        _say("noalloc accept", n, w1, vocab)
        args = [a.to(dev) for a in _inputs(n, w1, vocab, seed)]
        want = _call(lib, _lib, "rlt_speculative_accept", args, n, w1, vocab, dev, True)
        got = _call(lib, _lib, "rlt_speculative_accept_noalloc", args, n, w1, vocab, dev, False)
        for a, b in zip(got, want):
            assert torch.equal(a, b)
        ref = osamp.speculative_accept(*(a.cpu() for a in args))
        assert torch.equal(got[0], ref.tokens) and torch.equal(got[1], ref.accepted)


def test_noalloc_accept_rejects_sizes_beyond_its_array(pkg):
    import ctypes

    from vllm_rlt_amd import _lib

    lib = _lib.library()
    cap = lib.rlt_speculative_accept_noalloc_max_bytes()
    assert cap == 8 << 20
    n, w1, vocab = 4096, 32, 1 << 20
    assert lib.rlt_speculative_accept_workspace_size(n, w1, vocab) > cap
    null = ctypes.c_void_p(0)
    st = lib.rlt_speculative_accept_noalloc(null, null, null, null, null, null, n, w1, vocab,
                                            null, null, null, null, null)
    assert st == 3
