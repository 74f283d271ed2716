"""GPU parity of the hip decode / windowed / prefill attention against the oracle.

Cases follow the reference's own GPU tests: tests/test_attention.py:225-379
(mixed batches, online-softmax stability, packed prefill, split-KV decode with
batch invariance) and tests/test_attention_64bit.py:7-30 (64-bit offsets).
Tolerances: bf16 2e-2, f16 2e-3, f32 1e-4 (max-abs and rtol), as there.
"""

import numpy as np
import pytest
import torch

from oracle import paged_ref as ref

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2e-2, torch.float16: 2e-3, torch.float32: 1e-4}
CODE = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def np32(t):
    return t.detach().float().cpu().numpy()


def oracle_decode(q, k, v, tables, lengths, window=0):
    out = ref.paged_attention(np32(q), np32(k), np32(v), tables.cpu().numpy(),
                              lengths.cpu().numpy(), window=window)
    return torch.from_numpy(ref.round_to(out, CODE[q.dtype]))


def assert_close(actual, expected, dtype):
    tol = TOL[dtype]
    torch.testing.assert_close(actual.float().cpu(), expected.float(), atol=tol, rtol=tol)


def random_paged(lengths, heads, kv_heads, head_dim, dtype, device, block=16, seed=1):
    gen = torch.Generator().manual_seed(seed)
    pages = sum(-(-n // block) for n in lengths) + 1
    k = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype).to(device)
    v = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype).to(device)
    order = torch.randperm(pages, generator=gen).tolist()
    width = max(1, max(-(-n // block) for n in lengths))
    tables = torch.full((len(lengths), width), -1, dtype=torch.int32)
    for row, n in enumerate(lengths):
        ids = [order.pop() for _ in range(-(-n // block))]
        tables[row, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
    q = torch.randn(len(lengths), heads, head_dim, generator=gen).to(dtype).to(device)
    context = torch.tensor(lengths, dtype=torch.int32, device=device)
    return q, k, v, tables.to(device), context


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_split_kv_decode_matches_oracle_and_is_batch_invariant(gpu, dtype):
    from vllm_rlt.kernels.hip_attention import paged_attention

    lengths = [0, 1, 31, 32, 33, 511, 512, 513, 4097, 10000]
    q, k, v, tables, context = random_paged(lengths, 8, 4, 128, dtype, gpu)
    actual = paged_attention(q, k, v, tables, context)
    torch.cuda.synchronize()
    assert_close(actual, oracle_decode(q, k, v, tables, context), dtype)
    assert torch.count_nonzero(actual[0]) == 0
    for row in (1, 5, 8, 9):
        one = slice(row, row + 1)
        alone = paged_attention(q[one], k, v, tables[one], context[one])
        assert torch.equal(alone[0], actual[row])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [7, 32, 64, 96, 128, 256])
@pytest.mark.parametrize("heads,kv_heads", [(6, 2), (16, 16)])
def test_decode_shapes(gpu, dtype, head_dim, heads, kv_heads):
    from vllm_rlt.kernels.hip_attention import paged_attention

    lengths = [1, 5, 17, 100, 300, 700]
    q, k, v, tables, context = random_paged(lengths, heads, kv_heads, head_dim, dtype, gpu,
                                            block=16, seed=head_dim)
    actual = paged_attention(q, k, v, tables, context)
    assert_close(actual, oracle_decode(q, k, v, tables, context), dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [320, 512])
def test_decode_wide_heads_split_and_merge(gpu, dtype, head_dim):
    """Head dims above 256 (up to the 512 the entry point accepts): rows long
    enough for several splits, so the merge runs with 8 dims per lane."""
    from vllm_rlt.kernels.hip_attention import paged_attention

    lengths = [1, 64, 65, 300, 2000]
    q, k, v, tables, context = random_paged(lengths, 4, 2, head_dim, dtype, gpu, block=16,
                                            seed=head_dim)
    actual = paged_attention(q, k, v, tables, context)
    assert_close(actual, oracle_decode(q, k, v, tables, context), dtype)


@pytest.mark.parametrize("block", [2, 3, 5, 16, 32])
def test_decode_odd_block_sizes(gpu, block):
    from vllm_rlt.kernels.hip_attention import paged_attention

    lengths = [1, 2, 3, 70, 71, 333, 1500]
    q, k, v, tables, context = random_paged(lengths, 4, 2, 32, torch.float32, gpu, block=block,
                                            seed=block)
    actual = paged_attention(q, k, v, tables, context)
    assert_close(actual, oracle_decode(q, k, v, tables, context), torch.float32)


def test_decode_online_softmax_is_stable_with_large_scores(gpu):
    from vllm_rlt.kernels.hip_attention import paged_attention

    gen = torch.Generator().manual_seed(89)
    k = (torch.randn(30, 5, 1, 32, generator=gen) * 8).to(gpu)
    v = torch.randn(30, 5, 1, 32, generator=gen).to(gpu)
    table = torch.randperm(30, generator=gen)[:15].to(torch.int32)
    positions = [0, 31, 32, 70]
    tables = table.repeat(4, 1).to(gpu)
    context = torch.tensor([p + 1 for p in positions], dtype=torch.int32, device=gpu)
    q = (torch.randn(4, 2, 32, generator=gen) * 8).to(gpu)
    actual = paged_attention(q, k, v, tables, context)
    expected = oracle_decode(q, k, v, tables, context)
    torch.testing.assert_close(actual.cpu(), expected, atol=2e-4, rtol=2e-4)


@pytest.mark.parametrize("window", [1, 7, 16, 100, 5000])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_windowed_decode_matches_oracle(gpu, window, dtype):
    from vllm_rlt.kernels.hip_attention import HipPagedAttention

    lengths = [0, 1, 15, 16, 17, 250, 1000, 4097]
    q, k, v, tables, context = random_paged(lengths, 8, 8, 64, dtype, gpu, seed=window)
    actual = HipPagedAttention().windowed(q, k, v, tables, context, window)
    assert_close(actual, oracle_decode(q, k, v, tables, context, window=window), dtype)


def test_decode_strided_layer_view_of_5d_pool(gpu):
    """Kernels get ``cache[:, layer]`` of a [N, L, bs, H, D] pool (strided blocks)."""
    from vllm_rlt.kernels.hip_attention import paged_attention

    gen = torch.Generator().manual_seed(5)
    pool_k = torch.randn(40, 3, 16, 4, 64, generator=gen).to(torch.bfloat16).to(gpu)
    pool_v = torch.randn(40, 3, 16, 4, 64, generator=gen).to(torch.bfloat16).to(gpu)
    tables = torch.randperm(40, generator=gen)[:36].view(3, 12).to(torch.int32).to(gpu)
    context = torch.tensor([191, 17, 100], dtype=torch.int32, device=gpu)
    q = torch.randn(3, 8, 64, generator=gen).to(torch.bfloat16).to(gpu)
    for layer in range(3):
        k, v = pool_k[:, layer], pool_v[:, layer]
        actual = paged_attention(q, k, v, tables, context)
        assert_close(actual, oracle_decode(q, k, v, tables, context), torch.bfloat16)


def test_decode_uses_64bit_physical_offsets(gpu):
    """Block id 2048 x block stride 2**20 elements = offset 2**31 (exact)."""
    from vllm_rlt.kernels.hip_attention import paged_attention

    if torch.cuda.mem_get_info()[0] < 9 * 2**30:
        pytest.fail("the 64-bit offset case needs 9 GiB of free GPU memory")
    shape, strides = (2049, 1, 1, 16), (2**20, 16, 16, 1)
    key = torch.empty_strided(shape, strides, device=gpu, dtype=torch.float16)
    value = torch.empty_strided(shape, strides, device=gpu, dtype=torch.float16)
    key[0].zero_()
    value[0].fill_(-3)
    key[2048].fill_(1)
    expected = torch.arange(16, device=gpu, dtype=torch.float16).view(1, 1, 16)
    value[2048].copy_(expected)
    query = torch.ones((1, 1, 16), device=gpu, dtype=torch.float16)
    table = torch.tensor([[2048]], device=gpu, dtype=torch.int32)
    lengths = torch.tensor([1], device=gpu, dtype=torch.int32)
    actual = paged_attention(query, key, value, table, lengths)
    torch.cuda.synchronize()
    torch.testing.assert_close(actual, expected, rtol=0, atol=0)
    del key, value


def test_decode_more_rows_than_one_launch(gpu):
    """70,000 rows (one head, head_dim 32) with mixed lengths: the launcher
    splits the rows into launches of 65,472 (whole 64-row groups for the
    in-kernel longest-first ranking); every row must equal its own one-row
    decode (batch invariance) and a seeded subsample the oracle, including
    rows on both sides of the launch boundary."""
    from vllm_rlt.kernels.hip_attention import paged_attention

    rows, block = 70000, 16
    gen = torch.Generator().manual_seed(31)
    lengths = torch.randint(0, 300, (rows,), generator=gen, dtype=torch.int32)
    lengths[65470:65475] = torch.tensor([299, 0, 17, 160, 1], dtype=torch.int32)
    width = 19
    pool_blocks = 4096
    k = torch.randn(pool_blocks, block, 1, 32, generator=gen).to(torch.bfloat16).to(gpu)
    v = torch.randn(pool_blocks, block, 1, 32, generator=gen).to(torch.bfloat16).to(gpu)
    tables = torch.randint(0, pool_blocks, (rows, width), generator=gen,
                           dtype=torch.int32).to(gpu)
    q = torch.randn(rows, 1, 32, generator=gen).to(torch.bfloat16).to(gpu)
    context = lengths.to(gpu)
    out = paged_attention(q, k, v, tables, context)
    picks = sorted({0, 1, 65471, 65472, 65473, 65474, rows - 1,
                    *torch.randint(0, rows, (40,), generator=gen).tolist()})
    for r in picks:
        single = paged_attention(q[r : r + 1], k, v, tables[r : r + 1], context[r : r + 1])
        assert torch.equal(out[r : r + 1], single), r
    idx = torch.tensor(picks, device=gpu)
    want = oracle_decode(q[idx], k, v, tables[idx], context[idx])
    assert_close(out[idx], want, torch.bfloat16)


def test_decode_closed_forms(gpu):
    """Length 1 returns V exactly; constant keys return the mean of V."""
    from vllm_rlt.kernels.hip_attention import paged_attention

    gen = torch.Generator().manual_seed(3)
    k = torch.randn(8, 16, 2, 128, generator=gen).to(gpu)
    v = torch.randn(8, 16, 2, 128, generator=gen).to(gpu)
    tables = torch.tensor([[3, 5], [6, 1]], dtype=torch.int32, device=gpu)
    q = torch.randn(2, 2, 128, generator=gen).to(gpu)
    one = paged_attention(q, k, v, tables, torch.tensor([1, 1], dtype=torch.int32, device=gpu))
    torch.testing.assert_close(one[0], v[3, 0], rtol=0, atol=1e-6)
    torch.testing.assert_close(one[1], v[6, 0], rtol=0, atol=1e-6)
    k[5].fill_(0.25)
    k[3].fill_(0.25)
    lengths = torch.tensor([20, 20], dtype=torch.int32, device=gpu)
    out = paged_attention(q, k, v, tables, lengths)
    mean = torch.cat([v[3], v[5, :4]]).mean(0)
    torch.testing.assert_close(out[0], mean, atol=1e-5, rtol=1e-5)


PREFILL_CASES = [(37, 5), (100, 100), (3, 3), (130, 70), (129, 120)]


def prefill_inputs(sequences, heads, kv_heads, head_dim, dtype, device, seed=0):
    gen = torch.Generator().manual_seed(seed)
    block, blocks = 16, 96
    k = torch.randn(blocks, block, kv_heads, head_dim, generator=gen).to(dtype).to(device)
    v = torch.randn(blocks, block, kv_heads, head_dim, generator=gen).to(dtype).to(device)
    order = torch.randperm(blocks, generator=gen).tolist()
    width = max(-(-n // block) for n, _ in sequences)
    tables = torch.zeros(len(sequences), width, dtype=torch.int32)
    for s, (n, _) in enumerate(sequences):
        ids = [order.pop() for _ in range(-(-n // block))]
        tables[s, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
    total = sum(c for _, c in sequences)
    q = torch.randn(total, heads, head_dim, generator=gen).to(dtype).to(device)
    lengths = torch.tensor([n for n, _ in sequences], dtype=torch.int32, device=device)
    starts = [0]
    for _, c in sequences:
        starts.append(starts[-1] + c)
    cu = torch.tensor(starts, dtype=torch.int32, device=device)
    return q, k, v, tables.to(device), lengths, cu, max(c for _, c in sequences)


def oracle_prefill(q, k, v, tables, lengths, cu):
    out = ref.paged_prefill(np32(q), np32(k), np32(v), tables.cpu().numpy(),
                            lengths.cpu().numpy(), cu.cpu().numpy())
    return torch.from_numpy(ref.round_to(out, CODE[q.dtype]))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("head_dim,heads,kv_heads", [(64, 4, 2), (96, 8, 8), (128, 16, 16),
                                                     (32, 2, 1), (7, 2, 2)])
def test_packed_prefill_matches_per_query_oracle(gpu, dtype, head_dim, heads, kv_heads):
    from vllm_rlt.kernels.hip_attention import paged_prefill_attention

    q, k, v, tables, lengths, cu, max_q = prefill_inputs(PREFILL_CASES, heads, kv_heads,
                                                         head_dim, dtype, gpu)
    actual = paged_prefill_attention(q, k, v, tables, lengths, cu, max_q)
    assert_close(actual, oracle_prefill(q, k, v, tables, lengths, cu), dtype)


@pytest.mark.parametrize("block", [2, 4, 5, 8, 16, 32, 64])
@pytest.mark.parametrize("dtype,head_dim,heads,kv_heads", [(torch.bfloat16, 128, 4, 4),
                                                          (torch.float16, 64, 4, 2)])
def test_packed_prefill_block_sizes_and_long_tables(gpu, block, dtype, head_dim, heads, kv_heads):
    """MFMA tiles with every page-addressing path (power-of-two pages smaller and
    larger than a staging store's rows, non-power-of-two pages) and page tables
    longer than the 512-entry LDS segment (9000 keys: 141 to 4500 pages)."""
    from vllm_rlt.kernels.hip_attention import paged_prefill_attention

    sequences = [(9000, 130), (700, 300), (33, 33), (513, 1)]
    gen = torch.Generator().manual_seed(block)
    pages = sum(-(-n // block) for n, _ in sequences)
    k = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype).to(gpu)
    v = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype).to(gpu)
    order = torch.randperm(pages, generator=gen).tolist()
    width = max(-(-n // block) for n, _ in sequences)
    tables = torch.full((len(sequences), width), -1, dtype=torch.int32)
    for s, (n, _) in enumerate(sequences):
        ids = [order.pop() for _ in range(-(-n // block))]
        tables[s, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
    total = sum(c for _, c in sequences)
    q = torch.randn(total, heads, head_dim, generator=gen).to(dtype).to(gpu)
    cu = torch.tensor(np.cumsum([0] + [c for _, c in sequences]), dtype=torch.int32, device=gpu)
    lengths = torch.tensor([n for n, _ in sequences], dtype=torch.int32, device=gpu)
    tables = tables.to(gpu)
    actual = paged_prefill_attention(q, k, v, tables, lengths, cu, 300)
    assert_close(actual, oracle_prefill(q, k, v, tables, lengths, cu), dtype)


@pytest.mark.parametrize("dtype,head_dim,heads,kv_heads", [(torch.bfloat16, 128, 8, 8),
                                                          (torch.float16, 64, 8, 2)])
def test_packed_prefill_long_sequences_ragged_queries(gpu, dtype, head_dim, heads, kv_heads):
    """Long prefixes (up to 5000 keys) with ragged query counts and decode rows
    in one packed batch, bf16 MHA and f16 GQA; also replayed from a captured
    graph."""
    from vllm_rlt.kernels.hip_attention import paged_prefill_attention

    sequences = [(4000, 300), (3000, 512), (2500, 1), (5000, 129), (1500, 64), (1100, 2),
                 (300, 40)]
    gen = torch.Generator().manual_seed(23)
    block = 16
    pages = sum(-(-n // block) for n, _ in sequences)
    k = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype).to(gpu)
    v = torch.randn(pages, block, kv_heads, head_dim, generator=gen).to(dtype).to(gpu)
    order = torch.randperm(pages, generator=gen).tolist()
    width = max(-(-n // block) for n, _ in sequences)
    tables = torch.full((len(sequences), width), -1, dtype=torch.int32)
    for s, (n, _) in enumerate(sequences):
        ids = [order.pop() for _ in range(-(-n // block))]
        tables[s, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
    total = sum(c for _, c in sequences)
    q = torch.randn(total, heads, head_dim, generator=gen).to(dtype).to(gpu)
    cu = torch.tensor(np.cumsum([0] + [c for _, c in sequences]), dtype=torch.int32, device=gpu)
    lengths = torch.tensor([n for n, _ in sequences], dtype=torch.int32, device=gpu)
    tables = tables.to(gpu)
    expected = oracle_prefill(q, k, v, tables, lengths, cu)
    actual = paged_prefill_attention(q, k, v, tables, lengths, cu, 512)
    assert_close(actual, expected, dtype)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        paged_prefill_attention(q, k, v, tables, lengths, cu, 512)
    torch.cuda.current_stream().wait_stream(stream)
    with torch.cuda.graph(graph):
        captured = paged_prefill_attention(q, k, v, tables, lengths, cu, 512)
    for _ in range(3):
        captured.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, actual)


def test_packed_prefill_mixed_with_decode_rows(gpu):
    """WCPB shape in miniature: long chunks with prefixes and q_len = 1 rows."""
    from vllm_rlt.kernels.hip_attention import paged_prefill_attention

    sequences = [(600, 512), (1030, 6), (1, 1), (200, 1), (64, 64), (900, 130), (77, 1)]
    gen = torch.Generator().manual_seed(11)
    block = 16
    pages = sum(-(-n // block) for n, _ in sequences)
    k = torch.randn(pages, block, 16, 128, generator=gen).to(torch.bfloat16).to(gpu)
    v = torch.randn(pages, block, 16, 128, generator=gen).to(torch.bfloat16).to(gpu)
    order = torch.randperm(pages, generator=gen).tolist()
    width = max(-(-n // block) for n, _ in sequences)
    tables = torch.full((len(sequences), width), -1, dtype=torch.int32)
    for s, (n, _) in enumerate(sequences):
        ids = [order.pop() for _ in range(-(-n // block))]
        tables[s, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
    total = sum(c for _, c in sequences)
    q = torch.randn(total, 16, 128, generator=gen).to(torch.bfloat16).to(gpu)
    cu = torch.tensor(np.cumsum([0] + [c for _, c in sequences]), dtype=torch.int32, device=gpu)
    lengths = torch.tensor([n for n, _ in sequences], dtype=torch.int32, device=gpu)
    tables = tables.to(gpu)
    actual = paged_prefill_attention(q, k, v, tables, lengths, cu, 512)
    assert_close(actual, oracle_prefill(q, k, v, tables, lengths, cu), torch.bfloat16)
    # The decode rows run on a side stream forked from and joined back into the
    # current stream: a captured graph must reproduce the eager result on every
    # replay, with other eager work and synchronisations in between.
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        paged_prefill_attention(q, k, v, tables, lengths, cu, 512)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        captured = paged_prefill_attention(q, k, v, tables, lengths, cu, 512)
    for _ in range(3):
        captured.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, actual)
        paged_prefill_attention(q, k, v, tables, lengths, cu, 512)  # eager work in between


def test_empty_inputs(gpu):
    from vllm_rlt.kernels.hip_attention import paged_attention, paged_prefill_attention

    k = torch.zeros(2, 16, 2, 64, device=gpu)
    empty_q = torch.empty(0, 2, 64, device=gpu)
    tables = torch.zeros(0, 1, dtype=torch.int32, device=gpu)
    lengths = torch.zeros(0, dtype=torch.int32, device=gpu)
    assert paged_attention(empty_q, k, k, tables, lengths).shape == (0, 2, 64)
    cu = torch.zeros(1, dtype=torch.int32, device=gpu)
    assert paged_prefill_attention(empty_q, k, k, tables, lengths, cu, 1).shape == (0, 2, 64)
    # q heads not a multiple of kv heads (tests/test_attention.py:99-107)
    q3 = torch.ones(1, 3, 64, device=gpu)
    one_table = torch.zeros(1, 1, dtype=torch.int32, device=gpu)
    one_length = torch.ones(1, dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError, match="positive multiple"):
        paged_attention(q3, k, k, one_table, one_length)
    with pytest.raises(ValueError, match="positive multiple"):
        paged_prefill_attention(q3, k, k, one_table, one_length,
                                torch.tensor([0, 1], dtype=torch.int32, device=gpu), 1)


def test_prefill_without_workspace_runs_decode_rows_through_mfma_tiles(gpu):
    """The C ABI accepts no workspace: every sequence (also q_len = 1) then goes
    through the MFMA tiles; results match the routed (split-KV) path."""
    from vllm_rlt.kernels._hip import library
    from vllm_rlt.kernels.hip_attention import dtype_code, paged_prefill_attention

    sequences = [(300, 1), (37, 5), (1000, 1), (129, 120), (5, 1)]
    q, k, v, tables, lengths, cu, max_q = prefill_inputs(sequences, 8, 8, 128, torch.bfloat16,
                                                         gpu, seed=21)
    routed = paged_prefill_attention(q, k, v, tables, lengths, cu, max_q)
    out = torch.empty_like(q)
    lib = library()
    lib.check(lib.vrh_paged_prefill(
        dtype_code(q.dtype), out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
        tables.data_ptr(), lengths.data_ptr(), cu.data_ptr(), len(sequences), q.shape[0], max_q,
        8, 8, 128, 16, tables.shape[1], tables.stride(0), q.stride(0), q.stride(1),
        out.stride(0), out.stride(1), *k.stride()[:3], *v.stride()[:3], None, 0,
        torch.cuda.current_stream().cuda_stream), "vrh_paged_prefill")
    expected = oracle_prefill(q, k, v, tables, lengths, cu)
    assert_close(out, expected, torch.bfloat16)
    assert_close(routed, expected, torch.bfloat16)


@pytest.mark.parametrize("dtype,head_dim", [(torch.float32, 128), (torch.bfloat16, 48)])
def test_packed_prefill_fallback_ignores_padding_rows(gpu, dtype, head_dim):
    """A bucketed q longer than cu_seqlens_q[-1] on the per-row fallback (f32,
    and a head dim without MFMA tiles): the padding rows belong to no sequence
    and are skipped (they must not read past a table's padded entries); the
    valid rows match the oracle."""
    from vllm_rlt.kernels.hip_attention import paged_prefill_attention

    sequences = [(70, 5), (33, 25)]
    q, k, v, tables, lengths, cu, max_q = prefill_inputs(sequences, 4, 2, head_dim, dtype, gpu)
    tables[1, 3:] = -1  # pad past the 3 pages of 33 keys, as the metadata planner does
    padded = torch.cat([q, torch.randn(9, *q.shape[1:], device=gpu).to(dtype)])
    actual = paged_prefill_attention(padded, k, v, tables, lengths, cu, max_q)
    torch.cuda.synchronize()
    assert_close(actual[: q.shape[0]], oracle_prefill(q, k, v, tables, lengths, cu), dtype)


@pytest.mark.parametrize("layout", ["same_pool", "pools_of_different_depth", "head_major_v"])
@pytest.mark.parametrize("block", [16, 8])
def test_packed_prefill_strided_kv_views(gpu, layout, block):
    """MFMA prefill over K / V layer views whose strides differ from each other
    (K and V from pools with different layer counts, or V stored head-major and
    viewed as [N, bs, H, D]), against the per-query oracle; the staging then
    forms separate K and V addresses instead of one shared offset."""
    from vllm_rlt.kernels.hip_attention import paged_prefill_attention

    sequences = [(2000, 300), (700, 129), (64, 64), (300, 1)]
    heads, head_dim, dtype = 8, 128, torch.bfloat16
    gen = torch.Generator().manual_seed(block + len(layout))
    pages = sum(-(-n // block) for n, _ in sequences) + 3
    if layout == "same_pool":
        pool = torch.randn(pages, 2, 2, block, heads, head_dim, generator=gen).to(dtype).to(gpu)
        k, v = pool[:, 0, 1], pool[:, 1, 1]
    elif layout == "pools_of_different_depth":
        kp = torch.randn(pages, 2, block, heads, head_dim, generator=gen).to(dtype).to(gpu)
        vp = torch.randn(pages, 3, block, heads, head_dim, generator=gen).to(dtype).to(gpu)
        k, v = kp[:, 1], vp[:, 2]
    else:
        k = torch.randn(pages, block, heads, head_dim, generator=gen).to(dtype).to(gpu)
        v = torch.randn(pages, heads, block, head_dim, generator=gen).to(dtype).to(gpu)
        v = v.permute(0, 2, 1, 3)
    order = torch.randperm(pages, generator=gen).tolist()
    width = max(-(-n // block) for n, _ in sequences)
    tables = torch.full((len(sequences), width), -1, dtype=torch.int32)
    for s, (n, _) in enumerate(sequences):
        ids = [order.pop() for _ in range(-(-n // block))]
        tables[s, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
    total = sum(c for _, c in sequences)
    q = torch.randn(total, heads, head_dim, generator=gen).to(dtype).to(gpu)
    cu = torch.tensor(np.cumsum([0] + [c for _, c in sequences]), dtype=torch.int32, device=gpu)
    lengths = torch.tensor([n for n, _ in sequences], dtype=torch.int32, device=gpu)
    tables = tables.to(gpu)
    actual = paged_prefill_attention(q, k, v, tables, lengths, cu, 300)
    expected = oracle_prefill(q, k.contiguous(), v.contiguous(), tables, lengths, cu)
    assert_close(actual, expected, dtype)


@pytest.mark.parametrize("count", [64, 65, 130])
def test_packed_prefill_many_sequences(gpu, count):
    """Batches ranked inside the MFMA kernel (up to 64 sequences) and by the
    separate ordering kernel (more), with decode rows, short chunks and a few
    long ones in one batch, against the per-query oracle."""
    from vllm_rlt.kernels.hip_attention import paged_prefill_attention

    gen = torch.Generator().manual_seed(count)
    sequences = []
    for s in range(count):
        kind = s % 5
        if kind == 0:
            sequences.append((int(torch.randint(1, 400, (1,), generator=gen)), 1))
        elif kind == 4 and s < 20:
            n = int(torch.randint(300, 1200, (1,), generator=gen))
            sequences.append((n, int(torch.randint(129, min(n, 400), (1,), generator=gen))))
        else:
            n = int(torch.randint(2, 200, (1,), generator=gen))
            sequences.append((n, int(torch.randint(1, n + 1, (1,), generator=gen))))
    block, heads = 16, 4
    pages = sum(-(-n // block) for n, _ in sequences)
    k = torch.randn(pages, block, heads, 128, generator=gen).to(torch.bfloat16).to(gpu)
    v = torch.randn(pages, block, heads, 128, generator=gen).to(torch.bfloat16).to(gpu)
    order = torch.randperm(pages, generator=gen).tolist()
    width = max(-(-n // block) for n, _ in sequences)
    tables = torch.full((count, width), -1, dtype=torch.int32)
    for s, (n, _) in enumerate(sequences):
        ids = [order.pop() for _ in range(-(-n // block))]
        tables[s, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
    total = sum(c for _, c in sequences)
    q = torch.randn(total, heads, 128, generator=gen).to(torch.bfloat16).to(gpu)
    cu = torch.tensor(np.cumsum([0] + [c for _, c in sequences]), dtype=torch.int32, device=gpu)
    lengths = torch.tensor([n for n, _ in sequences], dtype=torch.int32, device=gpu)
    tables = tables.to(gpu)
    max_q = max(c for _, c in sequences)
    actual = paged_prefill_attention(q, k, v, tables, lengths, cu, max_q)
    assert_close(actual, oracle_prefill(q, k, v, tables, lengths, cu), torch.bfloat16)
