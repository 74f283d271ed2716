"""The allocation-free decode entry point (vrh_paged_decode_noalloc) through the
C ABI, checked against vrh_paged_decode with a caller workspace on the same
inputs: the kernels are shared, so the outputs must be bit-identical. Two
calls in a row, the second with fewer rows and shorter contexts, so the
second reads partials the first left in the shared scratch only where it
wrote them itself."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(rows, max_len, seed, dtype=torch.bfloat16, heads=16, dim=128, block=16):
    gen = torch.Generator().manual_seed(seed)
    lengths = torch.randint(0, max_len + 1, (rows,), generator=gen, dtype=torch.int32)
    lengths[0] = max_len
    width = -(-max_len // block)
    pool = rows * width + 3
    k = (torch.randn(pool, 2, block, heads, dim, generator=gen) * 0.5).to(dtype)
    v = (torch.randn(pool, 2, block, heads, dim, generator=gen) * 0.5).to(dtype)
    tables = torch.randperm(pool, generator=gen)[: rows * width].to(torch.int32).view(rows, width)
    q = (torch.randn(rows, heads, dim, generator=gen) * 0.5).to(dtype)
    dev = torch.device("cuda:0")
    return (q.to(dev), k.to(dev)[:, 1], v.to(dev)[:, 1], tables.to(dev), lengths.to(dev))


def _args(out, q, k, v, tables, lengths):
    from vllm_rlt.kernels.hip_attention import dtype_code

    return [dtype_code(q.dtype), out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
            tables.data_ptr(), lengths.data_ptr(), q.shape[0], q.shape[1], k.shape[2],
            q.shape[2], k.shape[1], tables.shape[1], tables.stride(0), q.stride(0), q.stride(1),
            out.stride(0), out.stride(1), *k.stride()[:3], *v.stride()[:3], 0]


def _run_both(lib, inputs):
    q = inputs[0]
    stream = torch.cuda.current_stream().cuda_stream
    want = torch.full_like(q, float("nan"))
    nbytes = lib.vrh_paged_decode_workspace_bytes(q.shape[0], q.shape[1], q.shape[2])
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    lib.check(lib.vrh_paged_decode(*_args(want, *inputs), workspace.data_ptr(), nbytes, stream),
              "vrh_paged_decode")
    got = torch.full_like(q, float("nan"))
    lib.check(lib.vrh_paged_decode_noalloc(*_args(got, *inputs), stream),
              "vrh_paged_decode_noalloc")
    torch.cuda.synchronize()
    return got, want


def test_noalloc_matches_workspace_decode_twice(gpu):
    from vllm_rlt.kernels._hip import library

    lib = library()
    print("noalloc: call 1, 64 rows up to 4096 tokens; call 2, 9 rows up to 700 tokens",
          flush=True)
    got, want = _run_both(lib, _inputs(64, 4096, seed=3))
    assert torch.equal(got, want)
    got, want = _run_both(lib, _inputs(9, 700, seed=4))
    assert torch.equal(got, want)


def test_noalloc_f32_window_and_gqa(gpu):
    from vllm_rlt.kernels._hip import library
    from vllm_rlt.kernels.hip_attention import paged_attention, paged_attention_noalloc

    library()
    print("noalloc: f32 GQA windowed decode, 5 rows", flush=True)
    q, k, v, tables, lengths = _inputs(5, 1000, seed=5, dtype=torch.float32, heads=4, dim=64)
    q = torch.cat([q, q], dim=1)  # 8 q heads over 4 kv heads
    for window in (0, 100):
        want = paged_attention(q, k, v, tables, lengths, window=window)
        out = torch.empty_like(q)
        got = paged_attention_noalloc(q, k, v, tables, lengths, window=window, out=out)
        torch.cuda.synchronize()
        assert got is out
        assert torch.equal(got, want)


def test_noalloc_grouped_query_mfma_twice(gpu):
    """Groups of 8 q heads per kv head (the MFMA decode kernel), bf16: two
    calls in a row, the second with fewer rows, against the workspace entry."""
    from vllm_rlt.kernels._hip import library
    from vllm_rlt.kernels.hip_attention import paged_attention, paged_attention_noalloc

    library()
    for rows, max_len, seed in ((24, 3000, 6), (5, 400, 7)):
        print(f"noalloc: bf16 32 q heads over 4 kv heads, {rows} rows up to {max_len} tokens",
              flush=True)
        q, k, v, tables, lengths = _inputs(rows, max_len, seed=seed, heads=4)
        q = q.repeat_interleave(8, dim=1).contiguous()
        want = paged_attention(q, k, v, tables, lengths)
        got = paged_attention_noalloc(q, k, v, tables, lengths)
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_noalloc_captured_in_a_graph_replays_like_eager(gpu):
    """The allocation-free entry point under HIP-graph capture: replayed three
    times, with eager decode calls on other inputs and synchronisations in
    between (they overwrite the shared scratch), every replay equals the
    eager result of the captured inputs."""
    from vllm_rlt.kernels._hip import library
    from vllm_rlt.kernels.hip_attention import paged_attention, paged_attention_noalloc

    lib = library()
    # resolves the scratch address of this device before capture
    assert lib.vrh_paged_decode_noalloc_max_bytes() == 96 << 20
    print("noalloc: graph capture, 48 rows up to 3000 tokens, 3 replays", flush=True)
    q, k, v, tables, lengths = _inputs(48, 3000, seed=8)
    other = _inputs(20, 2000, seed=9)
    want = paged_attention(q, k, v, tables, lengths)
    out = torch.full_like(q, float("nan"))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        paged_attention_noalloc(q, k, v, tables, lengths, out=out)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_attention_noalloc(q, k, v, tables, lengths, out=out)
    for _ in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        paged_attention_noalloc(*other)  # overwrites the scratch between replays
        torch.cuda.synchronize()


def test_noalloc_rejects_sizes_beyond_the_scratch(gpu):
    from vllm_rlt.kernels._hip import library

    lib = library()
    limit = lib.vrh_paged_decode_noalloc_max_bytes()
    assert limit == 96 << 20
    rows = 1
    while lib.vrh_paged_decode_workspace_bytes(rows, 16, 128) <= limit:
        rows += 1
    # Dangling pointers: the size check must refuse before any launch.
    dummy = ctypes.c_void_p(16)
    code = lib.vrh_paged_decode_noalloc(
        2, dummy, dummy, dummy, dummy, dummy, dummy, rows, 16, 16, 128, 16, 4, 4, 2048, 128,
        2048, 128, 32768, 2048, 128, 32768, 2048, 128, 0, None)
    assert code == 1
    assert b"built-in scratch" in lib.vrh_last_error()
