"""GPU parity of grouped-query decode against the oracle: groups of 3 and 5
to 16 q heads per kv head run on the MFMA kernel, groups of 4 (and 2) on the
VALU kernel with one wave serving the group.

Reference semantics: kernels/paged_attention.py:12-36 (kv head = h // G via
repeat_interleave, fp32 softmax, zero rows), its windowed variant (:39-71) and
the split-KV batch invariance of tests/test_attention.py:375-379. Tolerances
as the other decode tests: bf16 2e-2, f16 2e-3 (max-abs and rtol).
"""

import pytest
import torch

from test_gpu_attention import assert_close, oracle_decode, random_paged

pytestmark = pytest.mark.gpu

LENGTHS = [0, 1, 2, 15, 16, 17, 31, 33, 100, 511, 512, 513, 2047, 4097, 9000]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("heads,kv_heads", [(16, 4), (32, 8), (32, 4), (32, 2), (12, 2),
                                            (10, 2), (16, 1)])
def test_gqa_decode_matches_oracle(gpu, dtype, head_dim, heads, kv_heads):
    from vllm_rlt.kernels.hip_attention import paged_attention

    q, k, v, tables, context = random_paged(LENGTHS, heads, kv_heads, head_dim, dtype, gpu,
                                            seed=heads * 7 + kv_heads)
    actual = paged_attention(q, k, v, tables, context)
    assert_close(actual, oracle_decode(q, k, v, tables, context), dtype)
    assert torch.count_nonzero(actual[0]) == 0
    # batch invariance: a row alone gives the same bits as in the batch
    for row in (1, 9, 13, 14):
        one = slice(row, row + 1)
        alone = paged_attention(q[one], k, v, tables[one], context[one])
        assert torch.equal(alone[0], actual[row])


@pytest.mark.parametrize("window", [1, 9, 100, 3000])
def test_gqa_windowed_decode_matches_oracle(gpu, window):
    from vllm_rlt.kernels.hip_attention import HipPagedAttention

    q, k, v, tables, context = random_paged(LENGTHS, 32, 4, 128, torch.bfloat16, gpu,
                                            seed=window)
    actual = HipPagedAttention().windowed(q, k, v, tables, context, window)
    assert_close(actual, oracle_decode(q, k, v, tables, context, window=window), torch.bfloat16)


@pytest.mark.parametrize("block", [5, 8, 32, 64])
def test_gqa_decode_block_sizes(gpu, block):
    from vllm_rlt.kernels.hip_attention import paged_attention

    q, k, v, tables, context = random_paged(LENGTHS, 16, 2, 128, torch.bfloat16, gpu,
                                            block=block, seed=block)
    actual = paged_attention(q, k, v, tables, context)
    assert_close(actual, oracle_decode(q, k, v, tables, context), torch.bfloat16)


def test_gqa_decode_large_scores_are_stable(gpu):
    """Scores far above the running reference max (lazy rescale) and rows whose
    maximum appears late in the row."""
    from vllm_rlt.kernels.hip_attention import paged_attention

    q, k, v, tables, context = random_paged([700, 3000, 64], 32, 4, 128, torch.float16, gpu,
                                            seed=11)
    k = k.clone()
    k[tables[1, 150].item()] *= 24  # one page of very large keys late in row 1
    q = q * 4
    actual = paged_attention(q, k, v, tables, context)
    assert_close(actual, oracle_decode(q, k, v, tables, context), torch.float16)
    assert torch.isfinite(actual.float()).all()


def test_gqa_decode_packed_prefill_decode_rows(gpu):
    """Decode rows of a packed prefill call (the prefill entry point routes
    q_len = 1 sequences to the decode kernel) with grouped heads."""
    from vllm_rlt.kernels.hip_attention import paged_prefill_attention

    lengths = [900, 1, 40, 2500]
    q_lens = [1, 1, 1, 1]
    q, k, v, tables, context = random_paged(lengths, 16, 2, 128, torch.bfloat16, gpu, seed=5)
    cu = torch.tensor([0, 1, 2, 3, 4], dtype=torch.int32, device=gpu)
    actual = paged_prefill_attention(q, k, v, tables, context, cu, max(q_lens))
    assert_close(actual, oracle_decode(q, k, v, tables, context), torch.bfloat16)


def test_gqa_decode_graph_replays(gpu):
    """The MFMA path captured in a HIP graph: three replays, with eager work
    and synchronisations between them, each equal to the eager result."""
    from vllm_rlt.kernels.hip_attention import paged_attention

    q, k, v, tables, context = random_paged(LENGTHS, 32, 2, 128, torch.bfloat16, gpu, seed=21)
    eager = paged_attention(q, k, v, tables, context)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        paged_attention(q, k, v, tables, context)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = paged_attention(q, k, v, tables, context)
    for _ in range(3):
        captured.fill_(float("nan"))
        paged_attention(q[:3], k, v, tables[:3], context[:3])  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)
