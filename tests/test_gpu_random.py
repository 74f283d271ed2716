"""Seeded random decode and packed-prefill batches against the oracle.

Each case draws a dtype, head_dim (including dims without MFMA tiles), a
grouped-query ratio, a block size, row lengths (zero, one, short, long), an
optional window and, for decode, rows that share page prefixes with the row
before them. Decode must match the oracle (kernels/paged_attention.py:12-71)
within the decode tolerances and give a row alone the same bits as in the
batch (tests/test_attention.py:375-379); packed prefill must match the
per-query oracle (kernels/triton_attention.py:313-366). Tolerances: bf16 2e-2,
f16 2e-3, f32 1e-4.
"""

import random

import numpy as np
import pytest
import torch

from test_gpu_attention import assert_close, oracle_decode, oracle_prefill

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def draw_shape(rng):
    dtype = rng.choice(DTYPES)
    head_dim = rng.choice([32, 64, 96, 128, 80])
    kv_heads = rng.choice([1, 2, 4])
    group = rng.choice([1, 1, 2, 3, 4, 8, 16])
    block = rng.choice([1, 2, 5, 8, 16, 16, 32])
    return dtype, head_dim, kv_heads, kv_heads * group, block


def pool(gen, pages, block, kv_heads, head_dim, dtype, device):
    k = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype).to(device)
    v = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype).to(device)
    return k, v


@pytest.mark.parametrize("seed", range(16))
def test_random_decode(gpu, seed):
    from vllm_rlt.kernels.hip_attention import paged_attention

    rng = random.Random(seed)
    gen = torch.Generator().manual_seed(seed)
    dtype, head_dim, kv_heads, q_heads, block = draw_shape(rng)
    rows = rng.randint(1, 40)
    lengths = [rng.choice([0, 1, rng.randint(1, 40), rng.randint(1, 2000)]) for _ in range(rows)]
    window = rng.choice([0, 0, rng.randint(1, 400)])
    pages = [-(-n // block) for n in lengths]
    width = max(1, max(pages))
    total = sum(pages) + 2
    k, v = pool(gen, total, block, kv_heads, head_dim, dtype, gpu)
    free = torch.randperm(total, generator=gen).tolist()
    tables = torch.full((rows, width), -1, dtype=torch.int32)
    for r in range(rows):
        ids = [free.pop() for _ in range(pages[r])]
        if r > 0 and rng.random() < 0.5:  # share a prefix with the row before
            shared = min(pages[r], pages[r - 1], rng.randint(0, width))
            ids = tables[r - 1, :shared].tolist() + ids[shared:]
        if ids:
            tables[r, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
    q = torch.randn(rows, q_heads, head_dim, generator=gen).to(dtype).to(gpu)
    tables = tables.to(gpu)
    context = torch.tensor(lengths, dtype=torch.int32, device=gpu)
    actual = paged_attention(q, k, v, tables, context, window=window)
    assert_close(actual, oracle_decode(q, k, v, tables, context, window=window), dtype)
    for r in {0, rows // 2, rows - 1}:
        alone = paged_attention(q[r : r + 1], k, v, tables[r : r + 1], context[r : r + 1],
                                window=window)
        assert torch.equal(alone[0], actual[r]), f"row {r}"


@pytest.mark.parametrize("seed", range(16))
def test_random_packed_prefill(gpu, seed):
    from vllm_rlt.kernels.hip_attention import paged_prefill_attention

    rng = random.Random(1000 + seed)
    gen = torch.Generator().manual_seed(1000 + seed)
    dtype, head_dim, kv_heads, q_heads, block = draw_shape(rng)
    sequences = []
    for _ in range(rng.randint(1, 20)):
        n = rng.choice([1, rng.randint(1, 64), rng.randint(1, 700)])
        q_len = rng.choice([1, n, rng.randint(1, n), min(n, rng.randint(1, 140))])
        sequences.append((n, q_len))
    pages = [-(-n // block) for n, _ in sequences]
    total = sum(pages) + 1
    k, v = pool(gen, total, block, kv_heads, head_dim, dtype, gpu)
    free = torch.randperm(total, generator=gen).tolist()
    tables = torch.full((len(sequences), max(pages)), -1, dtype=torch.int32)
    for s, count in enumerate(pages):
        ids = [free.pop() for _ in range(count)]
        tables[s, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
    q = torch.randn(sum(c for _, c in sequences), q_heads, head_dim, generator=gen)
    q = q.to(dtype).to(gpu)
    cu = torch.tensor(np.cumsum([0] + [c for _, c in sequences]), dtype=torch.int32, device=gpu)
    lengths = torch.tensor([n for n, _ in sequences], dtype=torch.int32, device=gpu)
    tables = tables.to(gpu)
    actual = paged_prefill_attention(q, k, v, tables, lengths, cu, max(c for _, c in sequences))
    assert_close(actual, oracle_prefill(q, k, v, tables, lengths, cu), dtype)
