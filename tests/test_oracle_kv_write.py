"""Pins the KV write oracle: the e4m3 encoder against torch's cast, quantize_fp8 and
the FP8 scatter against the reference's known-answer tests, finalize against the
reference's finalize test and a per-element brute force."""

import numpy as np
import pytest
import torch

from oracle import kv_write as ow
from oracle.fp8 import FP8_E4M3_MAX, dequantize_fp8, quantize_fp8


def _torch_codes(x):
    return x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_encoder_matches_torch_on_every_half_value():
    # every finite float16 inside the e4m3 range: all binades, both signs, every tie
    h = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.float16)
    x = h.float()
    x = x[(x.abs() <= FP8_E4M3_MAX) | torch.isnan(x)]
    ours = ow.e4m3_encode(x.numpy())
    want = _torch_codes(x)
    nan = np.isnan(x.numpy())
    assert np.array_equal(ours[~nan], want[~nan])
    assert np.all((ours[nan] & 0x7F) == 0x7F)


def test_e4m3_encoder_matches_torch_on_random_floats():
    g = torch.Generator().manual_seed(0)
    x = (torch.rand(200000, generator=g) * 2 - 1) * torch.exp2(torch.randint(-24, 9, (200000,), generator=g).float())
    x = x.clamp(-FP8_E4M3_MAX, FP8_E4M3_MAX)
    assert np.array_equal(ow.e4m3_encode(x.numpy()), _torch_codes(x))


def test_e4m3_encoder_known_codes():
    # format facts: 448 = 0x7e, 2^-6 (smallest normal) = 0x08, 2^-9 (smallest subnormal)
    # = 0x01, half of it ties to 0, 1.0 = 0x38, -0.0 keeps its sign bit
    x = np.array([448.0, 2.0 ** -6, 2.0 ** -9, 2.0 ** -10, 1.0, -0.0, 1.0625, 1.1875],
                 dtype=np.float32)
    assert ow.e4m3_encode(x).tolist() == [0x7E, 0x08, 0x01, 0x00, 0x38, 0x80, 0x38, 0x3A]


def test_quantize_round_trip_bound_and_zero_vectors():
    # reference KAT: tests/test_fp8_kv_cache.py:46-55
    x = torch.randn(64, 4, 32) * torch.logspace(-3, 3, 64).view(64, 1, 1)
    codes, scale = quantize_fp8(x)
    error = (dequantize_fp8(codes, scale, torch.float32) - x).abs()
    assert (error <= x.abs().amax(-1, keepdim=True) / 16 + 1e-30).all()
    zeros = quantize_fp8(torch.zeros(2, 8))
    assert torch.isfinite(zeros[1]).all() and not dequantize_fp8(*zeros, torch.float32).any()
    # the scale is amax * float32(1/448) and each vector's amax maps to a code of 448
    assert torch.equal(scale, x.abs().amax(-1) * np.float32(1 / 448))
    assert bool((codes.float().abs().amax(-1) >= 416).all())


def test_fixed_scale_saturates():
    # reference KAT: tests/test_fa4_fp8.py:39-49
    x = torch.tensor([[0.25] * 64, [1000.0] * 64])
    codes, scale = quantize_fp8(x, 0.02)
    back = dequantize_fp8(codes, scale, torch.float32)
    torch.testing.assert_close(back[0], torch.full((64,), 0.24))
    torch.testing.assert_close(back[1], torch.full((64,), 448 * 0.02))


def _case(rows=10, pages=6, block=8, heads=2, dim=16, seed=0):
    g = torch.Generator().manual_seed(seed)
    slots = torch.randperm(pages * block, generator=g)[:rows]
    k = torch.randn(rows, heads, dim, generator=g)
    v = torch.randn(rows, heads, dim, generator=g)
    return slots // block, slots % block, k, v


@pytest.mark.parametrize("active", [None, 0, 7, 10])
def test_store_kv_skips_masked_inactive_and_outside_rows(active):
    blocks, offsets, k, v = _case()
    blocks[2] = 99          # outside the pool: skipped
    mask = torch.tensor([1, 0, 1, 1, 0, 1, 1, 1, 1, 1], dtype=torch.bool)
    kc, vc = torch.zeros(6, 8, 2, 16), torch.zeros(6, 8, 2, 16)
    act = None if active is None else torch.tensor(active, dtype=torch.int32)
    ow.store_kv(kc, vc, k, v, blocks, offsets, mask=mask, active=act)
    for i in range(10):
        written = bool(mask[i]) and i != 2 and (active is None or i < active)
        b, o = int(blocks[i]), int(offsets[i])
        if b >= 6:
            continue
        assert torch.equal(kc[b, o], k[i] if written else torch.zeros(2, 16))
        assert torch.equal(vc[b, o], v[i] if written else torch.zeros(2, 16))
    assert int((kc != 0).any(-1).any(-1).sum()) == sum(
        bool(mask[i]) and i != 2 and (active is None or i < active) for i in range(10))


@pytest.mark.parametrize("fixed_scale", [None, 0.02])
def test_store_fp8_scatters_quantize_fp8(fixed_scale):
    blocks, offsets, k, v = _case(seed=3)
    kc = torch.zeros(6, 8, 2, 16, dtype=torch.float8_e4m3fn)
    vc = kc.clone()
    ks, vs = torch.ones(6, 8, 2), torch.ones(6, 8, 2)
    mask = torch.ones(10, dtype=torch.bool)
    mask[4] = False
    ow.store_fp8(k, v, kc, vc, ks, vs, blocks, offsets, mask=mask, fixed_scale=fixed_scale)
    for x, c, s in ((k, kc, ks), (v, vc, vs)):
        want_c, want_s = quantize_fp8(x, fixed_scale)
        for i in range(10):
            b, o = int(blocks[i]), int(offsets[i])
            if i == 4:
                assert not c[b, o].float().any() and bool((s[b, o] == 1).all())
            else:
                assert torch.equal(c[b, o].view(torch.uint8), want_c[i].view(torch.uint8))
                assert torch.equal(s[b, o], want_s[i])


def _tables(slots, planes, width, nblocks, seed):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randperm(nblocks, generator=g)[: slots * planes * width]
    return ids.view(slots, planes, width).to(torch.int32)


def test_finalize_copies_exit_plane_into_deeper_planes_only():
    # the reference's finalize test (tests/test_fp8_kv_cache.py:142-152): position 5
    # exited at depth 0, every deeper plane then reads depth 0's entry in every layer
    slots, planes, width, page, layers, nblocks = 1, 4, 2, 4, 2, 8
    tables = _tables(slots, planes, width, nblocks, 0)
    pool = torch.randn(nblocks, layers, page, 2, 8)
    vpool = torch.randn(nblocks, layers, page, 2, 8)
    before_k, before_v = pool.clone(), vpool.clone()
    ow.finalize_rows(torch.tensor([[0, 0, 5]]), tables, pool, vpool, page)
    src = int(tables[0, 0, 1])
    for depth in range(1, planes):
        dst = int(tables[0, depth, 1])
        assert torch.equal(pool[dst, :, 1], before_k[src, :, 1])
        assert torch.equal(vpool[dst, :, 1], before_v[src, :, 1])
    # nothing else moved: other offsets, the exit plane, the other page
    changed = (pool != before_k).flatten(2).any(-1)
    assert set(map(tuple, changed.nonzero().tolist())) <= {
        (int(tables[0, d, 1]), layer) for d in range(1, planes) for layer in range(layers)}


def test_finalize_brute_force_over_many_descriptors():
    slots, planes, width, page, layers, nblocks = 3, 4, 3, 4, 3, 40
    tables = _tables(slots, planes, width, nblocks, 1)
    pool = torch.randn(nblocks, layers, page, 6)
    vpool = torch.randn(nblocks, layers, page, 6)
    # distinct (slot, position) pairs so copies never overlap; one at the deepest plane,
    # one out of range
    desc = torch.tensor([[0, 0, 3], [0, 2, 9], [1, 1, 0], [2, 3, 7], [2, 0, 11], [1, 0, 12]])
    k0, v0 = pool.clone(), vpool.clone()
    ow.finalize_rows(desc, tables, pool, vpool, page)
    want_k, want_v = k0.clone(), v0.clone()
    for slot, depth, pos in desc.tolist():
        if pos >= width * page:
            continue
        for t in range(depth + 1, planes):
            for layer in range(layers):
                for ch in range(6):
                    s = int(tables[slot, depth, pos // page])
                    d = int(tables[slot, t, pos // page])
                    want_k[d, layer, pos % page, ch] = k0[s, layer, pos % page, ch]
                    want_v[d, layer, pos % page, ch] = v0[s, layer, pos % page, ch]
    assert torch.equal(pool, want_k) and torch.equal(vpool, want_v)
