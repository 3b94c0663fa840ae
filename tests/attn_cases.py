"""Seeded synthetic paged-KV inputs shared by the attention tests and the bench.

A pool [num_blocks, layers, block_size, kv_heads, head_dim] is allocated like the
reference KV manager (vllm_rlt/core/kv_cache_manager.py:261-271) and one layer's
strided view [:, layer] is what the kernels read.  Each sequence (request x
plane) owns a random permutation slice of the pool's blocks.
"""

import math

import torch


def make_pool(num_blocks, layers, block_size, kv_heads, head_dim, dtype, g, layer=0, scale=1.0):
    shape = (num_blocks, layers, block_size, kv_heads, head_dim)
    if dtype == torch.float8_e4m3fn:
        k = (torch.randn(shape, generator=g) * 8).clamp(-448, 448).to(dtype)
        v = (torch.randn(shape, generator=g) * 8).clamp(-448, 448).to(dtype)
    else:
        k = (torch.randn(shape, generator=g) * scale).to(dtype)
        v = (torch.randn(shape, generator=g) * scale).to(dtype)
    return k, v, k[:, layer], v[:, layer]


def random_tables(lengths, block_size, num_blocks, g, width=None):
    need = [math.ceil(n / block_size) for n in lengths]
    width = width or max(max(need), 1)
    assert sum(need) <= num_blocks
    order = torch.randperm(num_blocks, generator=g).tolist()
    tables = torch.zeros(len(lengths), width, dtype=torch.int32)
    for r, c in enumerate(need):
        ids = [order.pop() for _ in range(c)]
        if ids:
            tables[r, :c] = torch.tensor(ids, dtype=torch.int32)
    return tables
