"""The torch operator library ``vllm_rlt._C`` (csrc/torch_ops.cpp).

CPU: the module loads through the reference's loader contract
(kernels/_extension.py:7-23), registers the reference's
``vllm_rlt::silu_and_mul`` schema (csrc/torch_bindings.cpp:6-14) and the
paged-KV ops, and has no CPU kernel (no silent host fallback).

GPU: every op gives bit-identical results to the ctypes adapter over the same
C entry point (also captured in a HIP graph and replayed), and its checks raise
RuntimeError (TORCH_CHECK), as the reference's native entry does (csrc/activation/silu_and_mul.cu:221-232).
"""

import pytest
import torch

from vllm_rlt.kernels import activation, hip_attention as hip
from vllm_rlt.kernels._extension import load_extension, try_load_extension

SCHEMAS = {
    "paged_attention": "vllm_rlt_hip::paged_attention(Tensor q, Tensor key_cache, "
    "Tensor value_cache, Tensor block_tables, Tensor context_lengths, int window=0) -> Tensor",
    "paged_prefill": "vllm_rlt_hip::paged_prefill(Tensor q, Tensor key_cache, Tensor value_cache, "
    "Tensor block_tables, Tensor context_lengths, Tensor cu_seqlens_q, int max_seqlen_q) -> Tensor",
    "kv_append": "vllm_rlt_hip::kv_append(Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor k, "
    "Tensor v, Tensor write_blocks, Tensor write_offsets, Tensor? write_mask=None, "
    "Tensor? active_rows=None) -> ()",
    "kv_gather": "vllm_rlt_hip::kv_gather(Tensor key_cache, Tensor value_cache, Tensor table, "
    "int length) -> (Tensor, Tensor)",
    "kv_finalize": "vllm_rlt_hip::kv_finalize(Tensor(a!) key_cache, Tensor(b!) value_cache, "
    "Tensor descriptors, Tensor tables, int planes) -> ()",
    "kv_copy_blocks": "vllm_rlt_hip::kv_copy_blocks(Tensor(a!) key_cache, Tensor(b!) value_cache, "
    "Tensor src_blocks, Tensor dst_blocks) -> ()",
}


def test_extension_registers_the_schemas():
    assert try_load_extension()
    load_extension()
    assert str(torch.ops.vllm_rlt.silu_and_mul.default._schema) == \
        "vllm_rlt::silu_and_mul(Tensor gate, Tensor up) -> Tensor"
    for name, schema in SCHEMAS.items():
        assert str(getattr(torch.ops.vllm_rlt_hip, name).default._schema) == schema


def test_ops_have_no_cpu_kernel():
    load_extension()
    gate = torch.zeros(4)
    with pytest.raises(NotImplementedError):
        torch.ops.vllm_rlt.silu_and_mul(gate, gate)
    q = torch.zeros(1, 1, 8)
    cache = torch.zeros(1, 1, 1, 8)
    with pytest.raises(NotImplementedError):
        torch.ops.vllm_rlt_hip.paged_attention(q, cache, cache, torch.zeros(1, 1, dtype=torch.int32),
                                               torch.zeros(1, dtype=torch.int32))


def _pool(gen, blocks, layers, bs, heads, dim, dtype, device):
    k = torch.randn(blocks, layers, bs, heads, dim, generator=gen).to(dtype).to(device)
    v = torch.randn(blocks, layers, bs, heads, dim, generator=gen).to(dtype).to(device)
    return k, v


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("q_heads", [16, 32])
def test_paged_attention_op_matches_adapter(gpu, dtype, q_heads):
    load_extension()
    gen = torch.Generator().manual_seed(3)
    kc, vc = _pool(gen, 96, 2, 16, 8, 128, dtype, gpu)
    rows = 9
    tables = torch.randperm(96, generator=gen)[:rows * 10].view(rows, 10).to(torch.int32).to(gpu)
    lengths = torch.tensor([0, 1, 15, 16, 17, 100, 159, 160, 77], dtype=torch.int32, device=gpu)
    q = torch.randn(rows, q_heads, 128, generator=gen).to(dtype).to(gpu)
    for window in (0, 33):
        want = hip.paged_attention(q, kc[:, 1], vc[:, 1], tables, lengths, window=window)
        got = torch.ops.vllm_rlt_hip.paged_attention(q, kc[:, 1], vc[:, 1], tables, lengths,
                                                     window)
        torch.cuda.synchronize()
        assert torch.equal(got, want)


@pytest.mark.gpu
def test_paged_prefill_op_matches_adapter(gpu):
    load_extension()
    gen = torch.Generator().manual_seed(4)
    kc, vc = _pool(gen, 128, 1, 16, 16, 128, torch.bfloat16, gpu)
    tables = torch.randperm(128, generator=gen)[:4 * 32].view(4, 32).to(torch.int32).to(gpu)
    lengths = torch.tensor([300, 1, 512, 45], dtype=torch.int32, device=gpu)
    cu = torch.tensor([0, 200, 201, 457, 502], dtype=torch.int32, device=gpu)
    q = torch.randn(502, 16, 128, generator=gen).to(torch.bfloat16).to(gpu)
    want = hip.paged_prefill_attention(q, kc[:, 0], vc[:, 0], tables, lengths, cu, 256)
    got = torch.ops.vllm_rlt_hip.paged_prefill(q, kc[:, 0], vc[:, 0], tables, lengths, cu, 256)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.gpu
def test_kv_ops_match_adapter(gpu):
    load_extension()
    gen = torch.Generator().manual_seed(5)
    base_k, base_v = _pool(gen, 64, 3, 16, 4, 64, torch.bfloat16, gpu)
    rows = 20
    blocks = torch.randperm(64, generator=gen)[:rows].to(torch.int64).to(gpu)
    offsets = torch.randint(0, 16, (rows,), generator=gen).to(torch.int64).to(gpu)
    k = torch.randn(rows, 4, 64, generator=gen).to(torch.bfloat16).to(gpu)
    v = torch.randn(rows, 4, 64, generator=gen).to(torch.bfloat16).to(gpu)
    mask = (torch.arange(rows) % 3 != 0).to(gpu)
    active = torch.tensor([17], dtype=torch.int32, device=gpu)
    a_k, a_v = base_k.clone(), base_v.clone()
    b_k, b_v = base_k.clone(), base_v.clone()
    hip.kv_append(a_k[:, 2], a_v[:, 2], k, v, blocks, offsets, write_mask=mask, active_rows=active)
    torch.ops.vllm_rlt_hip.kv_append(b_k[:, 2], b_v[:, 2], k, v, blocks, offsets, mask, active)
    torch.cuda.synchronize()
    assert torch.equal(a_k, b_k) and torch.equal(a_v, b_v)
    assert not torch.equal(a_k, base_k)

    table = torch.randperm(64, generator=gen)[:12].to(torch.int32).to(gpu)
    want = hip.kv_gather(a_k[:, 1], a_v[:, 1], table, 181)
    got = torch.ops.vllm_rlt_hip.kv_gather(a_k[:, 1], a_v[:, 1], table, 181)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])

    planes = 4
    tables = torch.randperm(64, generator=gen)[:2 * planes * 8].view(2 * planes, 8)
    tables = tables.to(torch.int32).to(gpu)
    desc = torch.tensor([[0, 1, 37], [1, 0, 5], [1, 3, 100]], dtype=torch.int64, device=gpu)
    hip.kv_finalize(a_k, a_v, desc, tables, planes)
    torch.ops.vllm_rlt_hip.kv_finalize(b_k, b_v, desc, tables, planes)
    torch.cuda.synchronize()
    assert torch.equal(a_k, b_k) and torch.equal(a_v, b_v)

    src = torch.tensor([3, 9, 40], dtype=torch.int64, device=gpu)
    dst = torch.tensor([10, 2, 63], dtype=torch.int64, device=gpu)
    hip.kv_copy_blocks(a_k, a_v, src, dst)
    torch.ops.vllm_rlt_hip.kv_copy_blocks(b_k, b_v, src, dst)
    torch.cuda.synchronize()
    assert torch.equal(a_k, b_k) and torch.equal(a_v, b_v)
    assert torch.equal(b_k[63], b_k[40])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_silu_and_mul_op_matches_adapter(gpu, dtype):
    load_extension()
    gen = torch.Generator().manual_seed(6)
    gate = (torch.randn(37, 1031, generator=gen) * 4).to(dtype).to(gpu)
    up = torch.randn(37, 1031, generator=gen).to(dtype).to(gpu)
    got = torch.ops.vllm_rlt.silu_and_mul(gate, up)
    assert torch.equal(got, activation.silu_and_mul(gate, up))
    assert torch.ops.vllm_rlt.silu_and_mul(gate[:0], up[:0]).shape == (0, 1031)


@pytest.mark.gpu
def test_op_checks_raise_runtime_error(gpu):
    load_extension()
    gate = torch.zeros(8, device=gpu)
    with pytest.raises(RuntimeError, match="same dtype"):
        torch.ops.vllm_rlt.silu_and_mul(gate, gate.half())
    with pytest.raises(RuntimeError, match="contiguous inputs"):
        torch.ops.vllm_rlt.silu_and_mul(torch.zeros(4, 4, device=gpu).t(),
                                        torch.zeros(4, 4, device=gpu).t())
    q = torch.zeros(2, 16, 128, dtype=torch.bfloat16, device=gpu)
    cache = torch.zeros(4, 16, 8, 128, dtype=torch.bfloat16, device=gpu)
    tables = torch.zeros(2, 4, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="context_lengths"):
        torch.ops.vllm_rlt_hip.paged_attention(q, cache, cache, tables,
                                               torch.zeros(2, dtype=torch.int64, device=gpu))
    with pytest.raises(RuntimeError, match="one row per query row"):
        torch.ops.vllm_rlt_hip.paged_attention(q, cache, cache, tables[:1],
                                               torch.zeros(1, dtype=torch.int32, device=gpu))


@pytest.mark.gpu
def test_ops_in_a_captured_graph(gpu):
    """The torch ops captured in one HIP graph (decode, prefill, append) and
    replayed three times, with new inputs written in place and eager work in
    between; every replay gives the eager result bit for bit."""
    load_extension()
    gen = torch.Generator().manual_seed(6)
    kc, vc = _pool(gen, 128, 1, 16, 8, 128, torch.bfloat16, gpu)
    k_view, v_view = kc[:, 0], vc[:, 0]
    tables = torch.randperm(128, generator=gen)[:4 * 30].view(4, 30).to(torch.int32).to(gpu)
    lengths = torch.tensor([300, 1, 450, 45], dtype=torch.int32, device=gpu)
    cu = torch.tensor([0, 200, 201, 457, 502], dtype=torch.int32, device=gpu)
    q_dec = torch.empty(4, 16, 128, dtype=torch.bfloat16, device=gpu)
    q_pre = torch.empty(502, 16, 128, dtype=torch.bfloat16, device=gpu)
    k_new = torch.empty(4, 8, 128, dtype=torch.bfloat16, device=gpu)
    v_new = torch.empty_like(k_new)
    blocks = tables[:, 0].to(torch.int64)
    offsets = torch.tensor([3, 0, 15, 7], dtype=torch.int64, device=gpu)

    def fill(seed):
        g = torch.Generator().manual_seed(seed)
        q_dec.copy_(torch.randn(q_dec.shape, generator=g).to(torch.bfloat16))
        q_pre.copy_(torch.randn(q_pre.shape, generator=g).to(torch.bfloat16))
        k_new.copy_(torch.randn(k_new.shape, generator=g).to(torch.bfloat16))
        v_new.copy_(torch.randn(v_new.shape, generator=g).to(torch.bfloat16))

    def step():
        torch.ops.vllm_rlt_hip.kv_append(k_view, v_view, k_new, v_new, blocks, offsets)
        dec = torch.ops.vllm_rlt_hip.paged_attention(q_dec, k_view, v_view, tables, lengths, 0)
        pre = torch.ops.vllm_rlt_hip.paged_prefill(q_pre, k_view, v_view, tables, lengths, cu, 256)
        return dec, pre

    fill(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dec_out, pre_out = step()
    for seed in (1, 2, 3):
        fill(seed)
        graph.replay()
        torch.cuda.synchronize()
        got_dec, got_pre = dec_out.clone(), pre_out.clone()
        want_dec, want_pre = step()  # eager, same inputs (the append rewrites the same slots)
        torch.cuda.synchronize()
        assert torch.equal(got_dec, want_dec), seed
        assert torch.equal(got_pre, want_pre), seed
        hip.paged_attention(q_dec, k_view, v_view, tables, lengths)  # eager work in between
