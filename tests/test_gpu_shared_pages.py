"""GPU parity of decode over rows whose page tables share pages with their
neighbours (parallel samples of one prompt, prefix-grouped batches).

The decode kernel reads pages that a neighbouring row also holds at the same
table index with cache-allocating loads and every other page with streaming
loads; only the cache policy depends on that, so each row must give the same
bits whether it is decoded with its sharing neighbours or alone (the split-KV
batch invariance of tests/test_attention.py:375-379), and match the oracle
(kernels/paged_attention.py:12-36) within the decode tolerances (bf16 2e-2,
f16 2e-3). The sharing patterns cover: prefixes that start at page 0 (shared
by 2-4 rows, ending inside and beyond a row's length), pages shared only past
page 0, identical tables with different lengths, zero-length rows inside a
group, block sizes that are not powers of two, windows, grouped-query heads
(VALU and MFMA kernels) and packed decode rows of a prefill batch.
"""

import pytest
import torch

from test_gpu_attention import assert_close, oracle_decode

pytestmark = pytest.mark.gpu


def shared_batch(heads, kv_heads, head_dim, dtype, device, block=16, seed=3):
    """Rows with the sharing patterns listed in the module docstring."""
    gen = torch.Generator().manual_seed(seed)
    next_page = [0]

    def fresh(count):
        ids = list(range(next_page[0], next_page[0] + count))
        next_page[0] += count
        return ids

    def pages(n):
        return -(-n // block)

    rows = []  # (table ids, length)
    # Group A: 4 rows share 40 pages from page 0; one row ends inside them.
    prefix = fresh(40)
    for n in (40 * block + 300, 40 * block + 1, 20 * block + 7, 40 * block + 999):
        own = max(0, pages(n) - 40)
        rows.append((prefix[: min(40, pages(n))] + fresh(own), n))
    # Group B: 2 rows share pages 10..29 but not page 0.
    mid = fresh(20)
    for n in (45 * block, 33 * block + 5):
        ids = fresh(10) + mid + fresh(pages(n) - 30)
        rows.append((ids, n))
    # A lone row.
    rows.append((fresh(pages(777)), 777))
    # Group C: 3 rows with one table, different lengths, and a zero-length row
    # between them.
    common = fresh(pages(3000))
    rows.append((common[: pages(3000)], 3000))
    rows.append(([], 0))
    rows.append((common[: pages(1500)], 1500))
    rows.append((common[: pages(17)], 17))
    # Group D: 2 rows share exactly one page (page 0), then diverge.
    first = fresh(1)
    for n in (9 * block + 3, 64 * block + 1):
        rows.append((first + fresh(pages(n) - 1), n))

    total = next_page[0] + 1
    perm = torch.randperm(total, generator=gen)
    width = max(1, max(len(ids) for ids, _ in rows))
    tables = torch.full((len(rows), width), -1, dtype=torch.int32)
    for r, (ids, _) in enumerate(rows):
        if ids:
            tables[r, : len(ids)] = perm[torch.tensor(ids)].to(torch.int32)
    k = torch.randn(total, block, kv_heads, head_dim, generator=gen).to(dtype).to(device)
    v = torch.randn(total, block, kv_heads, head_dim, generator=gen).to(dtype).to(device)
    q = torch.randn(len(rows), heads, head_dim, generator=gen).to(dtype).to(device)
    lengths = torch.tensor([n for _, n in rows], dtype=torch.int32, device=device)
    return q, k, v, tables.to(device), lengths


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads,kv_heads", [(16, 16), (32, 8), (64, 8)])
@pytest.mark.parametrize("block", [16, 5])
def test_shared_pages_match_oracle_and_rows_alone(gpu, dtype, heads, kv_heads, block):
    from vllm_rlt.kernels.hip_attention import paged_attention

    q, k, v, tables, lengths = shared_batch(heads, kv_heads, 128, dtype, gpu, block=block,
                                            seed=heads + block)
    actual = paged_attention(q, k, v, tables, lengths)
    assert_close(actual, oracle_decode(q, k, v, tables, lengths), dtype)
    assert torch.count_nonzero(actual[8]) == 0  # the zero-length row
    for row in range(q.shape[0]):
        one = slice(row, row + 1)
        alone = paged_attention(q[one], k, v, tables[one], lengths[one])
        assert torch.equal(alone[0], actual[row]), f"row {row}"


@pytest.mark.parametrize("window", [1, 100, 700])
def test_shared_pages_windowed(gpu, window):
    from vllm_rlt.kernels.hip_attention import HipPagedAttention

    q, k, v, tables, lengths = shared_batch(16, 16, 128, torch.bfloat16, gpu, seed=window)
    attn = HipPagedAttention()
    actual = attn.windowed(q, k, v, tables, lengths, window)
    assert_close(actual, oracle_decode(q, k, v, tables, lengths, window=window), torch.bfloat16)
    for row in (0, 3, 4, 7, 10):
        one = slice(row, row + 1)
        alone = attn.windowed(q[one], k, v, tables[one], lengths[one], window)
        assert torch.equal(alone[0], actual[row]), f"row {row}"


def test_shared_pages_packed_decode_rows(gpu):
    """One-query sequences of a packed prefill batch (decode rows routed to the
    split-KV kernel, table row = sequence) with shared tables."""
    from vllm_rlt.kernels.hip_attention import paged_attention, paged_prefill_attention

    q, k, v, tables, lengths = shared_batch(16, 16, 128, torch.bfloat16, gpu, seed=21)
    seqs = q.shape[0]
    cu = torch.arange(seqs + 1, dtype=torch.int32, device=gpu)
    packed = paged_prefill_attention(q, k, v, tables, lengths, cu, 1)
    assert_close(packed, oracle_decode(q, k, v, tables, lengths), torch.bfloat16)
    assert torch.equal(packed, paged_attention(q, k, v, tables, lengths))
