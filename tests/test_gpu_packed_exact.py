"""Packed rows reproduce single-query decode bit for bit (the reference's
``packed_matches_decode`` capability, attention/backend.py:21-23, relied on by
speculative verification, worker/speculative.py:176-178).

A packed call whose sequences all have at most 8 queries (max_seqlen_q <= 8)
runs every query as a split-KV decode row; query i of sequence s must equal,
with ``torch.equal``, the decode of a row with the same q, the same table row
and length n_s - q_s + i + 1. Lengths span the decode's 128-token split
boundaries and its one-split / multi-split cases; values are also checked
against the oracle so that equality is not agreement on a wrong answer.
"""

import numpy as np
import pytest
import torch

from oracle import paged_ref as ref

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 2e-2, torch.float16: 2e-3, torch.float32: 1e-4}
CODE = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}
BLOCK = 16


def np32(t):
    return t.detach().float().cpu().numpy()


def packed_batch(q_lens, lengths, heads, kv_heads, head_dim, dtype, device, seed):
    gen = torch.Generator().manual_seed(seed)
    pages = sum(-(-n // BLOCK) for n in lengths) + 3
    k = torch.randn(pages, BLOCK, kv_heads, head_dim, generator=gen).to(dtype).to(device)
    v = torch.randn(pages, BLOCK, kv_heads, head_dim, generator=gen).to(dtype).to(device)
    order = torch.randperm(pages, generator=gen).tolist()
    width = max(-(-n // BLOCK) for n in lengths) + 2
    tables = torch.full((len(lengths), width), -1, dtype=torch.int32)
    for s, n in enumerate(lengths):
        ids = [order.pop() for _ in range(-(-n // BLOCK))]
        tables[s, : len(ids)] = torch.tensor(ids, dtype=torch.int32)
    cu = torch.tensor([0, *np.cumsum(q_lens).tolist()], dtype=torch.int32)
    q = torch.randn(int(cu[-1]), heads, head_dim, generator=gen).to(dtype).to(device)
    return q, k, v, tables.to(device), torch.tensor(lengths, dtype=torch.int32,
                                                   device=device), cu.to(device)


def serial_rows(tables, lengths, cu):
    """Per-query decode rows of a packed batch: (table rows, lengths)."""
    rows, lens = [], []
    cu, n = cu.tolist(), lengths.tolist()
    for s in range(len(n)):
        q_len = cu[s + 1] - cu[s]
        for i in range(q_len):
            rows.append(s)
            lens.append(n[s] - q_len + i + 1)
    return (tables[torch.tensor(rows, device=tables.device)].contiguous(),
            torch.tensor(lens, dtype=torch.int32, device=tables.device))


CASES = [
    # (q_lens, context lengths): split boundaries at 128-token multiples,
    # one-split rows, 16-split rows, q_len 1..8
    ([1, 2, 3, 4, 5, 6, 7, 8], [8, 127, 129, 256, 260, 1000, 2049, 4100]),
    ([8] * 6 + [1] * 4, [8, 135, 136, 137, 2055, 3000, 1, 129, 128, 4096]),
    ([3, 5, 2, 8, 1], [20, 300, 130, 8200, 64]),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("groups", [1, 8])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_packed_rows_equal_serial_decode(gpu, dtype, groups, case):
    from vllm_rlt.kernels.hip_attention import paged_attention, paged_prefill_attention

    q_lens, lengths = CASES[case]
    kv_heads = 2
    heads = kv_heads * groups
    print(f"packed==decode: case {case} dtype {dtype} groups {groups}", flush=True)
    q, k, v, tables, context, cu = packed_batch(q_lens, lengths, heads, kv_heads, 128, dtype,
                                                gpu, seed=40 + case)
    packed = paged_prefill_attention(q, k, v, tables, context, cu, max(q_lens))
    rows, lens = serial_rows(tables, context, cu)
    serial = paged_attention(q, k, v, rows, lens)
    one_by_one = torch.cat([paged_attention(q[j : j + 1], k, v, rows[j : j + 1], lens[j : j + 1])
                            for j in range(q.shape[0])])
    torch.cuda.synchronize()
    assert torch.equal(packed, serial)
    assert torch.equal(packed, one_by_one)
    want = ref.paged_attention(np32(q), np32(k), np32(v), rows.cpu().numpy(), lens.cpu().numpy())
    torch.testing.assert_close(packed.float().cpu(),
                               torch.from_numpy(ref.round_to(want, CODE[dtype])),
                               atol=TOL[dtype], rtol=TOL[dtype])


def test_torch_op_packed_rows_equal_decode(gpu):
    """The registered torch operator gives the same exact rows."""
    from vllm_rlt.kernels._extension import load_extension
    from vllm_rlt.kernels.hip_attention import paged_attention

    load_extension()
    q_lens, lengths = CASES[0]
    q, k, v, tables, context, cu = packed_batch(q_lens, lengths, 16, 16, 128, torch.bfloat16,
                                                gpu, seed=7)
    packed = torch.ops.vllm_rlt_hip.paged_prefill(q, k, v, tables, context, cu, 8)
    rows, lens = serial_rows(tables, context, cu)
    serial = paged_attention(q, k, v, rows, lens)
    torch.cuda.synchronize()
    assert torch.equal(packed, serial)


def test_backend_declares_the_bound(gpu):
    from vllm_rlt.attention.backend import BackendCapabilities, create_backend

    backend = create_backend("hip", gpu, torch.bfloat16, 128, 16,
                             required_capabilities=BackendCapabilities(packed_prefill=True))
    assert backend.capabilities.packed_matches_decode
    assert backend.info["packed_matches_decode_max_seqlen_q"] == 8
    q_lens, lengths = [2, 8, 1], [40, 700, 3000]
    q, k, v, tables, context, cu = packed_batch(q_lens, lengths, 16, 16, 128, torch.bfloat16,
                                                gpu, seed=3)
    packed = backend.prefill(q, k, v, tables, context, cu, 8)
    rows, lens = serial_rows(tables, context, cu)
    assert torch.equal(packed, backend(q, k, v, rows, lens))


def test_packed_rows_equal_decode_many_sequences(gpu):
    """100 sequences of 1-8 queries (more than the 64 the prefill ranks in
    its kernel): still every packed query equals its decode row."""
    from vllm_rlt.kernels.hip_attention import paged_attention, paged_prefill_attention

    gen = torch.Generator().manual_seed(77)
    q_lens = torch.randint(1, 9, (100,), generator=gen).tolist()
    q_lens[0] = 8
    lengths = [max(q, n) for q, n in zip(q_lens, torch.randint(1, 3000, (100,),
                                                                 generator=gen).tolist())]
    print("packed==decode: 100 sequences", flush=True)
    q, k, v, tables, context, cu = packed_batch(q_lens, lengths, 16, 16, 128, torch.bfloat16,
                                                gpu, seed=78)
    packed = paged_prefill_attention(q, k, v, tables, context, cu, 8)
    rows, lens = serial_rows(tables, context, cu)
    serial = paged_attention(q, k, v, rows, lens)
    torch.cuda.synchronize()
    assert torch.equal(packed, serial)


def test_packed_exact_call_under_graph_capture(gpu):
    """A verification-shaped packed call (max_seqlen_q <= 8) captured in a HIP
    graph: every replay, with eager calls on other inputs in between, equals
    the eager result bit for bit."""
    from vllm_rlt.kernels.hip_attention import paged_prefill_attention

    q_lens, lengths = CASES[1]
    q, k, v, tables, context, cu = packed_batch(q_lens, lengths, 16, 16, 128, torch.bfloat16,
                                                gpu, seed=90)
    other = packed_batch(CASES[0][0], CASES[0][1], 16, 16, 128, torch.bfloat16, gpu, seed=91)
    want = paged_prefill_attention(q, k, v, tables, context, cu, 8)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        paged_prefill_attention(q, k, v, tables, context, cu, 8)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = paged_prefill_attention(q, k, v, tables, context, cu, 8)
    print("packed==decode: graph replays", flush=True)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        paged_prefill_attention(*other, 8)
        torch.cuda.synchronize()
