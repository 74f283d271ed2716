"""GPU parity of the kernels beside the attention path against the oracle:
SiLU-and-Mul (bit-exact against the float64 expression rounded as torch rounds
it), hidden-state row / segment movement and the batched snapshot / restore
offload (byte-exact).

Cases follow the reference's tests/test_activation.py (shapes, tails, storage
offsets, every 16-bit gate pattern, special values, graph replay, the error
contract) and the routing callers (worker/async_state.py:104-123,
worker/model_runner.py:515-597, core/kv_cache_manager.py:481-523).
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import activation_ref as act
from oracle import paged_ref as ref

pytestmark = pytest.mark.gpu

DTYPES = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def expected_silu(gate, up):
    dtype = DTYPES[gate.dtype]
    out = act.silu_and_mul(gate.float().cpu().numpy(), up.float().cpu().numpy(), dtype)
    return torch.from_numpy(np.array(out, dtype=np.float32, ndmin=1)).reshape(gate.shape)


def assert_bits_equal(actual, expected):
    """Equal values with equal bits (NaN only needs to be NaN)."""
    a = actual.float().cpu().flatten()
    e = expected.float().flatten()
    nan = torch.isnan(e)
    assert torch.equal(torch.isnan(a), nan)
    assert torch.equal(a[~nan].view(torch.int32), e[~nan].view(torch.int32))


def shifted(values, offset, device):
    """A contiguous view of `values` whose storage starts `offset` elements in."""
    storage = torch.empty(values.numel() + offset, dtype=values.dtype, device=device)
    view = storage[offset:].view(values.shape)
    view.copy_(values)
    return view


# ------------------------------------------------------------ SiLU-and-Mul
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize(
    "shape", [(), (0, 7), (2, 0), (1,), (7,), (8,), (9,), (3, 7), (2, 3, 9), (3, 5633), (128, 5632)]
)
@pytest.mark.parametrize("offsets", [(0, 0), (1, 0), (0, 1), (1, 3)])
def test_silu_and_mul_shapes_tails_and_offsets(gpu, dtype, shape, offsets):
    from vllm_rlt.kernels.activation import silu_and_mul

    gen = torch.Generator().manual_seed(42)
    count = math.prod(shape)
    gate = shifted(torch.randn(shape, generator=gen).to(dtype) * 4, offsets[0], gpu)
    up = shifted(torch.randn(shape, generator=gen).to(dtype), offsets[1], gpu)
    gate_before, up_before = gate.clone(), up.clone()
    out = silu_and_mul(gate, up)
    assert out.shape == gate.shape and out.dtype == dtype and out.device == gate.device
    assert_bits_equal(out, expected_silu(gate, up))
    assert torch.equal(gate, gate_before) and torch.equal(up, up_before)
    if count:
        assert out.data_ptr() not in (gate.data_ptr(), up.data_ptr())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_silu_and_mul_every_alignment_pair(gpu, dtype):
    from vllm_rlt.kernels.activation import silu_and_mul

    elements = 16 // torch.empty((), dtype=dtype).element_size()
    gen = torch.Generator().manual_seed(7)
    for count in [*range(2 * elements + 2), 17 * elements - 1, 17 * elements + 1, 4099]:
        g = torch.randn(count, generator=gen).to(dtype) * 6
        u = torch.randn(count, generator=gen).to(dtype)
        want = expected_silu(g, u)
        for go in range(elements):
            for uo in range(elements):
                out = silu_and_mul(shifted(g, go, gpu), shifted(u, uo, gpu))
                assert_bits_equal(out, want)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("offsets", [(0, 0), (1, 3)])
def test_silu_and_mul_every_gate_pattern(gpu, dtype, offsets):
    # tests/test_activation.py:360-430: all 16-bit gate patterns times factors
    # that cover signs, zeros, subnormals, extremes, inf and NaN.
    from vllm_rlt.kernels.activation import silu_and_mul

    info = torch.finfo(dtype)
    subnormal = info.tiny / (1024 if dtype == torch.float16 else 128)
    factors = torch.tensor([0.0, -0.0, 1.0, -1.0, 0.5, -2.0, info.tiny, subnormal, info.max,
                            -info.max, float("inf"), float("nan")], dtype=dtype)
    patterns = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(dtype)
    gate = patterns.repeat(factors.numel())
    up = factors.repeat_interleave(patterns.numel())
    out = silu_and_mul(shifted(gate, offsets[0], gpu), shifted(up, offsets[1], gpu))
    assert_bits_equal(out, expected_silu(gate, up))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_silu_and_mul_special_values(gpu, dtype):
    from vllm_rlt.kernels.activation import silu_and_mul

    info = torch.finfo(dtype)
    values = [float("nan"), float("inf"), -float("inf"), -100, -90, -85, -12, -1, -0.0, 0.0, 1,
              12, 100, info.tiny, info.tiny / 128, info.max, -info.max]
    v = torch.tensor(values, dtype=dtype)
    gate, up = torch.meshgrid(v, v, indexing="ij")
    gate, up = gate.contiguous(), up.contiguous()
    out = silu_and_mul(gate.to(gpu), up.to(gpu))
    assert_bits_equal(out, expected_silu(gate, up))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_silu_and_mul_large_misaligned_grid_stride(gpu, dtype):
    from vllm_rlt.kernels.activation import silu_and_mul

    gen = torch.Generator().manual_seed(3)
    count = 4096 * 256 * 8 + 5  # more vectors than one pass of the capped grid
    g = torch.randn(count, generator=gen).to(dtype) * 5
    u = torch.randn(count, generator=gen).to(dtype)
    out = silu_and_mul(shifted(g, 1, gpu), shifted(u, 3, gpu))
    assert_bits_equal(out, expected_silu(g, u))


def test_silu_and_mul_graph_replay_and_current_stream(gpu):
    from vllm_rlt.kernels.activation import silu_and_mul

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        gate = shifted(torch.randn(4097, dtype=torch.bfloat16), 1, gpu)
        up = shifted(torch.randn(4097, dtype=torch.bfloat16), 3, gpu)
        for _ in range(3):
            silu_and_mul(gate, up)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = silu_and_mul(gate, up)
    for fill in (3.0, -2.5, 0.75):
        gate.fill_(fill)
        up.fill_(2.0)
        graph.replay()
        torch.cuda.synchronize()
        assert_bits_equal(out, expected_silu(gate, up))


def test_silu_and_mul_error_contract(gpu):
    from vllm_rlt.kernels.activation import silu_and_mul

    with pytest.raises(ValueError, match="same shape"):
        silu_and_mul(torch.ones(2, 7, device=gpu), torch.ones(1, 7, device=gpu))
    with pytest.raises(TypeError, match="same dtype"):
        silu_and_mul(torch.ones(7, device=gpu), torch.ones(7, device=gpu, dtype=torch.float16))
    with pytest.raises(TypeError, match="supports float32"):
        silu_and_mul(torch.ones(7, device=gpu, dtype=torch.float64),
                     torch.ones(7, device=gpu, dtype=torch.float64))
    gate, up = torch.randn(2, 14, device=gpu).chunk(2, dim=-1)
    with pytest.raises(RuntimeError, match="contiguous inputs"):
        silu_and_mul(gate, up)
    g = torch.randn(16, device=gpu, requires_grad=True)
    with pytest.raises(RuntimeError, match="inference-only"):
        silu_and_mul(g, torch.randn_like(g))
    with torch.no_grad():
        out = silu_and_mul(g, torch.ones_like(g))
        assert not out.requires_grad
        assert_bits_equal(out, expected_silu(g.detach(), torch.ones_like(g)))


# ------------------------------------------------------- hidden-state rows
@pytest.mark.parametrize("dtype,width", [(torch.bfloat16, 2048), (torch.float32, 7),
                                          (torch.int64, 1), (torch.bfloat16, 4099)])
def test_gather_and_scatter_rows(gpu, dtype, width):
    from vllm_rlt.kernels.routing import gather_rows, scatter_rows

    gen = torch.Generator().manual_seed(11)
    pool = (torch.randn(50, width, generator=gen) * 100).to(dtype).to(gpu)
    slots = torch.randperm(50, generator=gen)[:40].to(gpu)
    out = torch.full((40, width), 7, dtype=dtype, device=gpu)
    gather_rows(pool, slots, out, 29)
    expect = ref.gather_rows(pool.cpu().numpy() if dtype != torch.bfloat16 else
                             pool.cpu().view(torch.int16).numpy(), slots.cpu().numpy(), 29, 40)
    got = out.cpu().view(torch.int16).numpy() if dtype == torch.bfloat16 else out.cpu().numpy()
    assert np.array_equal(got, expect)
    # scatter through a strided batch view (row stride > width)
    wide = (torch.randn(40, width + 5, generator=gen) * 100).to(dtype).to(gpu)
    values = wide[:, :width]
    target = pool.clone()
    scatter_rows(values, slots, target, 33)
    want = pool.clone()
    want[slots[:33]] = values[:33]
    assert torch.equal(target, want)


@pytest.mark.parametrize("dtype,width", [(torch.bfloat16, 2048), (torch.float32, 13)])
def test_gather_and_scatter_segments(gpu, dtype, width):
    from vllm_rlt.kernels.routing import gather_segments, scatter_segments

    gen = torch.Generator().manual_seed(5)
    slots, pool_rows = 6, 40
    pool = (torch.randn(slots * pool_rows, width, generator=gen) * 10).to(dtype).to(gpu)
    segs = [(3, 0, 17, 0, 1), (0, 5, 1, 17, 0), (5, 20, 20, 18, 1), (1, 39, 1, 38, 1),
            (2, 0, 0, 39, 1)]
    segments = torch.tensor(segs, dtype=torch.int64, device=gpu)
    batch = torch.zeros(39, width, dtype=dtype, device=gpu)
    gather_segments(pool, segments, batch, pool_rows, 20)
    view = (lambda t: t.cpu().view(torch.int16).numpy()) if dtype == torch.bfloat16 else \
        (lambda t: t.cpu().numpy())
    want = np.zeros_like(view(batch))
    ref.gather_segments(view(pool), np.array(segs), want, pool_rows)
    assert np.array_equal(view(batch), want)
    values = (torch.randn(39, width, generator=gen) * 10).to(dtype).to(gpu)
    target = pool.clone()
    scatter_segments(values, segments, target, pool_rows, 20)
    want_pool = view(pool).copy()
    ref.scatter_segments(view(values), np.array(segs), want_pool, pool_rows)
    assert np.array_equal(view(target), want_pool)


# --------------------------------------------------- snapshot / restore offload
def test_blocks_to_and_from_pinned_host(gpu):
    from vllm_rlt.kernels.hip_attention import kv_blocks_from_host, kv_blocks_to_host

    gen = torch.Generator().manual_seed(9)
    shape = (40, 3, 16, 4, 32)
    key_pool = torch.randn(shape, generator=gen).to(torch.bfloat16).to(gpu)
    value_pool = torch.randn(shape, generator=gen).to(torch.bfloat16).to(gpu)
    blocks = [31, 2, 17, 17, 39, 0]
    index = torch.tensor(blocks, dtype=torch.int64, device=gpu)
    host_k = torch.empty((6, *shape[1:]), dtype=torch.bfloat16, pin_memory=True)
    host_v = torch.empty_like(host_k, pin_memory=True)
    kv_blocks_to_host(key_pool, value_pool, index, host_k, host_v)
    torch.cuda.synchronize()
    want_k, want_v = ref.blocks_to_host(key_pool.cpu().view(torch.int16).numpy(),
                                        value_pool.cpu().view(torch.int16).numpy(), blocks)
    assert np.array_equal(host_k.view(torch.int16).numpy(), want_k)
    assert np.array_equal(host_v.view(torch.int16).numpy(), want_v)
    # restore into other blocks of fresh pools
    dest = [5, 6, 7, 8, 9, 10]
    k2, v2 = torch.zeros_like(key_pool), torch.zeros_like(value_pool)
    kv_blocks_from_host(k2, v2, torch.tensor(dest, device=gpu), host_k, host_v)
    torch.cuda.synchronize()
    expect_k = np.zeros_like(want_k, shape=key_pool.shape)
    expect_v = np.zeros_like(expect_k)
    ref.blocks_from_host(expect_k, expect_v, dest, want_k, want_v)
    assert np.array_equal(k2.cpu().view(torch.int16).numpy(), expect_k)
    assert np.array_equal(v2.cpu().view(torch.int16).numpy(), expect_v)


def test_offload_rejects_pageable_host_memory(gpu):
    from vllm_rlt.kernels import _hip
    from vllm_rlt.kernels.hip_attention import kv_blocks_to_host

    pool = torch.zeros((4, 2, 16, 2, 8), dtype=torch.bfloat16, device=gpu)
    index = torch.tensor([1, 2], device=gpu)
    pageable = torch.empty((2, 2, 16, 2, 8), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="pinned"):
        kv_blocks_to_host(pool, pool, index, pageable, pageable)
    # the C ABI itself refuses a pageable pointer before launching anything
    lib = _hip.library()
    buf = ctypes.create_string_buffer(4096)
    code = lib.vrh_kv_blocks_to_host(pool.data_ptr(), pool.data_ptr(), pool.stride(0) * 2,
                                     pool[0].numel() * 2, index.data_ptr(), ctypes.addressof(buf),
                                     ctypes.addressof(buf), 2,
                                     torch.cuda.current_stream().cuda_stream)
    assert code != 0 and b"pinned" in lib.vrh_last_error()
