"""GPU parity of the KV write side: the HIP writers against the oracle, bit for bit.

Mirrors the reference's tests/test_fp8_kv_cache.py:304-380 (FP8 store bitwise equal to
quantize_fp8, masked and inactive rows skipped) and :142-152 (finalize into deeper
planes), plus the plain scatter writers and a full e4m3 conversion sweep.
"""

from types import SimpleNamespace

import pytest
import torch

from oracle import kv_write as ow
from oracle.fp8 import FP8_E4M3_MAX, quantize_fp8

pytestmark = pytest.mark.gpu


def _slots(pages, block, rows, seed, device):
    g = torch.Generator().manual_seed(seed)
    s = torch.randperm(pages * block, generator=g)[:rows]
    return (s // block).to(device), (s % block).to(device)


def _bits(t):
    return t.view(torch.uint8) if t.element_size() == 1 else t.view(
        {2: torch.int16, 4: torch.int32}[t.element_size()])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16,
                                   torch.float8_e4m3fn])
@pytest.mark.parametrize("head_dim", [128, 5])
def test_store_kv_matches_index_put(pkg, dev, dtype, head_dim):
    pages, layers, block, heads, rows, layer = 12, 3, 16, 4, 40, 2
    shape = (pages, layers, block, heads, head_dim)
    kc = torch.zeros(shape, dtype=dtype, device=dev)
    vc = torch.zeros(shape, dtype=dtype, device=dev)
    blocks, offsets = _slots(pages, block, rows, 1, dev)
    k = torch.randn(rows, heads, head_dim, device=dev).to(dtype)
    # V strided across heads, a slice of a wider projection
    v = torch.randn(rows, heads, 2 * head_dim, device=dev).to(dtype)[..., :head_dim]
    pkg.store_kv(kc[:, layer], vc[:, layer], k, v, blocks, offsets)
    want_k, want_v = torch.zeros_like(kc).cpu(), torch.zeros_like(vc).cpu()
    ow.store_kv(want_k[:, layer], want_v[:, layer], k.cpu(), v.cpu(), blocks.cpu(), offsets.cpu())
    torch.cuda.synchronize()
    assert torch.equal(_bits(kc.cpu()), _bits(want_k))
    assert torch.equal(_bits(vc.cpu()), _bits(want_v))


@pytest.mark.parametrize("active", [0, 7, 10])
def test_masked_and_graph_writers_skip_rows(pkg, dev, active):
    pages, block, heads, dim, rows = 6, 8, 2, 64, 10
    kc = torch.zeros(pages, block, heads, dim, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    blocks, offsets = _slots(pages, block, rows, 4, dev)
    blocks[9] = pages + 3  # outside the pool: skipped
    k = torch.randn(rows, heads, dim, device=dev, dtype=torch.bfloat16)
    v = torch.randn(rows, heads, dim, device=dev, dtype=torch.bfloat16)
    mask = torch.tensor([1, 0, 1, 1, 0, 1, 1, 1, 1, 1], device=dev, dtype=torch.bool)
    count = torch.tensor(active, device=dev, dtype=torch.int32)
    batch = SimpleNamespace(write_blocks=blocks, write_offsets=offsets, write_mask=mask,
                            active_rows=count)
    pkg.write_graph_kv(kc, vc, batch, k, v)
    want_k, want_v = torch.zeros_like(kc).cpu(), torch.zeros_like(vc).cpu()
    ow.store_kv(want_k, want_v, k.cpu(), v.cpu(), blocks.cpu(), offsets.cpu(), mask=mask.cpu(),
                active=active)
    assert torch.equal(kc.cpu(), want_k) and torch.equal(vc.cpu(), want_v)
    kc.zero_(), vc.zero_()
    pkg.masked_kv_store(kc, vc, k, v, SimpleNamespace(write_blocks=blocks, write_offsets=offsets,
                                                      write_mask=mask))
    want_k.zero_(), want_v.zero_()
    ow.store_kv(want_k, want_v, k.cpu(), v.cpu(), blocks.cpu(), offsets.cpu(), mask=mask.cpu())
    assert torch.equal(kc.cpu(), want_k) and torch.equal(vc.cpu(), want_v)


@pytest.mark.parametrize("fixed_scale", [None, 0.02])
@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("head_dim", [128, 64, 256, 5])
def test_store_fp8_matches_quantize_fp8_bitwise(pkg, dev, fixed_scale, src, head_dim):
    torch.manual_seed(2)
    pages, layers, block, heads, rows, layer = 12, 3, 8, 4, 40, 1
    shape = (pages, layers, block, heads, head_dim)
    codes = [torch.zeros(shape, device=dev, dtype=torch.float8_e4m3fn) for _ in range(2)]
    scales = [torch.ones(shape[:-1], device=dev) for _ in range(2)]
    blocks, offsets = _slots(pages, block, rows, 2, dev)
    # float16 holds neither 1e-30 nor 1e4 * randn
    lo, hi = (-30, 4) if src != torch.float16 else (-4, 3)
    magnitudes = torch.logspace(lo, hi, rows, device=dev).view(rows, 1, 1)
    k = (torch.randn(rows, heads, head_dim, device=dev) * magnitudes).to(src)
    k[3] = 0  # a zero vector keeps a finite scale and zero codes
    v = torch.randn(rows, heads, 2 * head_dim, device=dev).to(src)[..., :head_dim]
    pkg.store_fp8(k, v, *(t[:, layer] for t in codes), *(t[:, layer] for t in scales), blocks,
                  offsets, FP8_E4M3_MAX, fixed_scale=fixed_scale)
    untouched = torch.ones(shape[:-1], dtype=torch.bool, device=dev)
    untouched[blocks, layer, offsets] = False
    for x, code, scale in zip((k, v), codes, scales):
        want_codes, want_scale = quantize_fp8(x.cpu(), fixed_scale)
        got = code[blocks, layer, offsets].cpu()
        assert torch.equal(got.view(torch.uint8), want_codes.view(torch.uint8))
        assert torch.equal(scale[blocks, layer, offsets].cpu().view(torch.int32),
                           want_scale.view(torch.int32))
        assert not code.float()[untouched].any() and bool((scale[untouched] == 1).all())


@pytest.mark.parametrize("fixed_scale", [None, 0.02])
@pytest.mark.parametrize("active", [0, 7, 10])
def test_store_fp8_skips_masked_and_inactive_rows(pkg, dev, fixed_scale, active):
    torch.manual_seed(4)
    pages, block, heads, dim, rows = 6, 8, 2, 64, 10
    shape = (pages, block, heads, dim)
    codes = [torch.zeros(shape, device=dev, dtype=torch.float8_e4m3fn) for _ in range(2)]
    scales = [torch.ones(shape[:-1], device=dev) for _ in range(2)]
    blocks, offsets = _slots(pages, block, rows, 5, dev)
    k = torch.randn(rows, heads, dim, device=dev, dtype=torch.bfloat16)
    v = torch.randn(rows, heads, dim, device=dev, dtype=torch.bfloat16)
    mask = torch.tensor([1, 0, 1, 1, 0, 1, 1, 1, 1, 1], device=dev, dtype=torch.bool)
    count = torch.tensor(active, device=dev, dtype=torch.int32)
    pkg.store_fp8(k, v, *codes, *scales, blocks, offsets, FP8_E4M3_MAX, mask=mask, active=count,
                  fixed_scale=fixed_scale)
    written = mask.clone()
    written[active:] = False
    for x, code, scale in zip((k, v), codes, scales):
        want_codes, want_scale = quantize_fp8(x.cpu(), fixed_scale)
        w = written.cpu()
        got = code[blocks, offsets].cpu()
        assert torch.equal(got[w].view(torch.uint8), want_codes[w].view(torch.uint8))
        assert torch.equal(scale[blocks, offsets].cpu()[w], want_scale[w])
        assert not got[~w].float().any()
        assert bool((scale[blocks, offsets].cpu()[~w] == 1).all())


def test_e4m3_conversion_sweep_matches_torch_cast(pkg, dev):
    # every float16 bit pattern as one element, stored with a fixed scale of 1: the codes
    # are the clamped value's e4m3fn cast (NaN kept, +-inf saturated by the clamp)
    h = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.float16)
    x = h.view(-1, 1, 256)
    rows = x.shape[0]
    codes = torch.zeros(rows, 1, 1, 256, dtype=torch.float8_e4m3fn, device=dev)
    scale = torch.ones(rows, 1, 1, device=dev)
    idx = torch.arange(rows, device=dev)
    zero = torch.zeros_like(idx)
    vc, vs = codes.clone(), scale.clone()
    pkg.store_fp8(x.to(dev), x.to(dev), codes, vc, scale, vs, idx, zero, FP8_E4M3_MAX,
                  fixed_scale=1.0)
    want, _ = quantize_fp8(x, 1.0)
    got = codes.view(rows, 1, 256).cpu().view(torch.uint8)
    want = want.view(torch.uint8)
    nan = torch.isnan(x.float())
    assert torch.equal(got[~nan], want[~nan])
    assert bool(((got[nan] & 0x7F) == 0x7F).all())
    # the independent format-definition encoder agrees too
    finite = ~nan
    assert torch.equal(got[finite], torch.from_numpy(
        ow.e4m3_encode(x.float().clamp(-448, 448)[finite].numpy())))


def test_store_fp8_nan_rows_keep_nan(pkg, dev):
    k = torch.randn(2, 1, 64, device=dev)
    k[0, 0, 7] = float("nan")
    codes = torch.zeros(2, 1, 1, 64, dtype=torch.float8_e4m3fn, device=dev)
    scale = torch.ones(2, 1, 1, device=dev)
    idx = torch.arange(2, device=dev)
    zero = torch.zeros_like(idx)
    pkg.store_fp8(k, k, codes, codes.clone(), scale, scale.clone(), idx, zero, FP8_E4M3_MAX)
    want_c, want_s = quantize_fp8(k.cpu())
    assert torch.equal(codes.view(2, 1, 64).cpu().float().isnan(), want_c.float().isnan())
    assert torch.isnan(scale[0]).all() and torch.equal(scale[1, 0].cpu(), want_s[1])


def _finalize_case(dev, dtype, tail, seed):
    g = torch.Generator().manual_seed(seed)
    slots, planes, width, page, layers, nblocks = 6, 4, 5, 16, 3, 160
    tables = torch.randperm(nblocks, generator=g)[: slots * planes * width]
    tables = tables.view(slots, planes, width).to(torch.int32)
    tables[4, 2, 4] = -1  # an unallocated page: nothing is copied into it
    shape = (nblocks, layers, page, *tail)
    k = torch.randn(shape, generator=g).to(dtype)
    v = torch.randn(shape, generator=g).to(dtype)
    pos = torch.randperm(width * page, generator=g)[:10]
    desc = torch.stack([torch.arange(10) % slots, torch.randint(0, planes, (10,), generator=g),
                        pos], 1)
    desc[3, 2] = width * page + 2  # outside the table: skipped
    desc[4] = torch.tensor([4, 1, 4 * page + 3])  # slot 4 appears in no other row
    return desc, tables, k, v, page


@pytest.mark.parametrize("dtype,tail", [(torch.bfloat16, (4, 128)), (torch.float32, (4,)),
                                        (torch.float8_e4m3fn, (4, 128)),
                                        (torch.float16, (3, 5))])
def test_finalize_matches_host_copy(pkg, dev, dtype, tail):
    desc, tables, k, v, page = _finalize_case(dev, dtype, tail, 7)
    kg, vg = k.to(dev), v.to(dev)
    pkg.finalize_rows(desc.to(dev), tables.to(dev), kg, vg, page)
    ow.finalize_rows(desc, tables, k, v, page)
    assert torch.equal(_bits(kg.cpu()), _bits(k)) and torch.equal(_bits(vg.cpu()), _bits(v))


def test_config_sized_write_round_trip(pkg, dev):
    # the verify window of the bench workload: 160 rows, 4 KV heads x 128, bf16, 16-token
    # pages; reading the written slots back returns the rows bit for bit
    pages, block, heads, dim, rows = 4096, 16, 4, 128, 160
    kc = torch.zeros(pages, block, heads, dim, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    blocks, offsets = _slots(pages, block, rows, 9, dev)
    k = torch.randn(rows, heads, dim, device=dev, dtype=torch.bfloat16)
    v = torch.randn(rows, heads, dim, device=dev, dtype=torch.bfloat16)
    pkg.store_kv(kc, vc, k, v, blocks, offsets)
    assert torch.equal(kc[blocks, offsets], k) and torch.equal(vc[blocks, offsets], v)
    assert int((kc != 0).any(-1).any(-1).sum()) == rows
