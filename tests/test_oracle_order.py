"""The C order model (oracle/order.c) against torch itself, bit for bit.

This pins the two torch-CPU summation orders the bit-exact acceptance contract
rests on (fp32 ``sum(-1)`` and sequential fp64 ``cumsum`` + right bisect),
which the GPU kernels reproduce.
"""

import numpy as np
import pytest
import torch

from oracle import order

SIZES = [1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 31, 32, 33, 63, 64, 100, 511, 512, 513, 4095, 4096,
         4097, 8191, 8192, 8193, 12345, 49152, 65536, 70001, 131072 + 5]


def _rows(V, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(6, V, generator=g)
    x[0] = x[0] ** 8  # heavily skewed
    x[1] = x[1] * 1e-38  # subnormal range
    x[2] = torch.randn(V, generator=g) * 1e6  # mixed signs, cancellation
    x[3] = torch.softmax(torch.randn(V, generator=g) * 3, -1)  # a probability row
    x[4] = (x[4] < 0.01).float() * x[4]  # sparse
    return x


@pytest.mark.parametrize("V", SIZES)
def test_row_sum_model_matches_torch_cpu_bitwise(V):
    x = _rows(V, V)
    want = x.sum(-1, dtype=torch.float32).numpy()
    got = order.row_sums(x.numpy())
    assert np.array_equal(want.view(np.int32), got.view(np.int32))


def test_row_sum_model_on_3d_verify_layout():
    # p.sum(-1) over [n, W1 + 1, V] (the call at speculative_sampling.py:138)
    g = torch.Generator().manual_seed(3)
    p = torch.softmax(torch.randn(8, 5, 49152, generator=g) * 3, -1)
    want = p.sum(-1, dtype=torch.float32).reshape(-1).numpy()
    got = order.row_sums(p.reshape(-1, 49152).numpy())
    assert np.array_equal(want.view(np.int32), got.view(np.int32))


def test_row_sum_model_nonfinite_rows():
    x = torch.rand(3, 1000)
    x[0, 17] = float("nan")
    x[1, 900] = float("inf")
    x[2, 5] = float("inf")
    x[2, 6] = float("-inf")
    want = x.sum(-1, dtype=torch.float32).numpy()
    got = order.row_sums(x.numpy())
    assert np.array_equal(np.isnan(want), np.isnan(got))
    ok = ~np.isnan(want)
    assert np.array_equal(want[ok], got[ok])


def _torch_categorical(w, u):
    c = w.double().cumsum(-1)
    m = c[:, -1]
    t = torch.minimum(u.double() * m, torch.nextafter(m, torch.zeros_like(m)))
    idx = torch.searchsorted(c, t[:, None], right=True).squeeze(-1)
    valid = torch.isfinite(m) & (m > 0)
    return torch.where(valid, idx, torch.zeros_like(idx)).clamp(0, w.shape[1] - 1), valid


@pytest.mark.parametrize("V", [1, 2, 7, 300, 2049])
def test_categorical_model_matches_torch(V):
    g = torch.Generator().manual_seed(V)
    w = torch.rand(64, V, generator=g) ** 4
    w[w < 0.2] = 0
    w[3] = 0
    w[5, 0] = float("nan")
    w[6, -1] = float("inf")
    u = torch.rand(64, generator=g)
    u[7] = 1.0
    u[8] = 0.0
    want_i, want_v = _torch_categorical(w, u)
    got_i, got_v = order.categorical(w.numpy(), u.numpy())
    assert np.array_equal(want_v.numpy(), got_v)
    assert np.array_equal(want_i.numpy(), got_i)


def test_categorical_model_negative_weights_follow_torch_bisect():
    # Out of contract (non-monotone cdf): the model replays torch's upper_bound.
    g = torch.Generator().manual_seed(11)
    w = torch.randn(40, 50, generator=g)
    w[:, 0] = 30.0  # keep mass positive
    u = torch.rand(40, generator=g)
    want_i, _ = _torch_categorical(w, u)
    got_i, _ = order.categorical(w.numpy(), u.numpy())
    assert np.array_equal(want_i.numpy(), got_i)


def test_import_guard_fixture_matches_torch_and_the_model(pkg):
    """The package's import-time sum-order guard: the committed fixture sums equal the C
    order model's and this host's torch's (the guard then reports a match)."""
    from vllm_rlt_amd import sampling

    assert sampling.CPU_SUM_ORDER_MATCHES
    for vocab, bits in sampling.ORDER_FIXTURE_SUMS.items():
        x = sampling.order_fixture(vocab)[None]
        got = order.row_sums(x)
        assert (int(got.view(np.int32)[0]) & 0xFFFFFFFF) == bits, vocab


@pytest.mark.parametrize("threads", [1, 2, 3, 5, 8])
def test_sum_1d_model_matches_torch_cpu_bitwise(threads):
    """``x.sum()`` of a whole 1-D tensor (the residual total of the synchronous runner,
    vllm_rlt/worker/speculative.py:66): serial below 32768 elements, else thread chunks."""
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        for V in (100, 32767, 32768, 32769, 49152, 65536, 65537, 151936, 300001):
            g = torch.Generator().manual_seed(V + threads)
            x = torch.rand(V, generator=g) ** 8
            want = x.sum()
            got = order.sum_1d(x.numpy(), threads)
            assert np.float32(want.item()).view(np.int32) == got.view(np.int32), V
    finally:
        torch.set_num_threads(prev)


def test_sum_1d_thread_chunks_change_the_bits():
    """The chunked order is not the row order: the model would catch a dropped chunking."""
    g = torch.Generator().manual_seed(5)
    differ = 0
    for _ in range(20):
        x = (torch.rand(151936, generator=g) ** 8).numpy()
        differ += order.sum_1d(x, 8).view(np.int32) != order.sum_1d(x, 1).view(np.int32)
    assert differ > 0
