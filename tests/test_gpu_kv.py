"""GPU parity of the bit-exact KV kernels (append, gather, finalize, block copy,
address expansion, routing metadata) against the oracle: exact equality.

Cases follow the reference: kv append with write_mask / active_rows
(kernels/routing.py:180-225, kernels/graph_kv.py:7-65, tests/test_cuda_graph.py:451),
LAST_EXITED finalize (kernels/routing.py:147-177, tests/test_kv_cache.py:38-58),
read (kv_cache_manager.py:834-854), and the integer routing kernels.
"""

import numpy as np
import pytest
import torch

from oracle import paged_ref as ref

pytestmark = pytest.mark.gpu


def pool(shape, dtype, device, seed):
    gen = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=gen).to(dtype).to(device)


def as_np(t):
    """Bit-preserving host copy (bf16 viewed as int16)."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.numpy().copy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("heads,head_dim", [(16, 128), (2, 7), (4, 96), (1, 1)])
@pytest.mark.parametrize("mode", ["plain", "mask", "active", "both"])
def test_append_is_bit_exact(gpu, dtype, heads, head_dim, mode):
    from vllm_rlt.kernels.hip_attention import kv_append

    key_pool = pool((30, 3, 16, heads, head_dim), dtype, gpu, 0)
    value_pool = pool((30, 3, 16, heads, head_dim), dtype, gpu, 1)
    rows = 37
    gen = torch.Generator().manual_seed(2)
    slots = torch.randperm(30 * 16, generator=gen)[:rows]
    blocks, offsets = slots // 16, slots % 16
    # k/v as non-contiguous row views of a fused projection output
    qkv = pool((rows, 3 * heads, head_dim), dtype, gpu, 3)
    k, v = qkv[:, heads : 2 * heads], qkv[:, 2 * heads :]
    mask = torch.rand(rows, generator=gen) > 0.3
    active = torch.tensor(29, dtype=torch.int32)
    use_mask = mode in ("mask", "both")
    use_active = mode in ("active", "both")
    layer = 1
    expected_k, expected_v = as_np(key_pool[:, layer]), as_np(value_pool[:, layer])
    ref.kv_append(expected_k, expected_v, as_np(k), as_np(v), blocks.numpy(), offsets.numpy(),
                  write_mask=mask.numpy() if use_mask else None,
                  active_rows=int(active) if use_active else None)
    kv_append(key_pool[:, layer], value_pool[:, layer], k, v, blocks.to(gpu), offsets.to(gpu),
              write_mask=mask.to(gpu) if use_mask else None,
              active_rows=active.to(gpu) if use_active else None)
    assert np.array_equal(as_np(key_pool[:, layer]), expected_k)
    assert np.array_equal(as_np(value_pool[:, layer]), expected_v)
    # other layers untouched
    assert np.array_equal(as_np(key_pool[:, 0]), as_np(pool((30, 3, 16, heads, head_dim), dtype,
                                                            gpu, 0)[:, 0]))


def test_append_many_rows_and_layers_in_one_launch(gpu):
    from vllm_rlt.kernels.hip_attention import kv_append_layers

    layers, rows = 24, 70000  # rows > 65535 exercises grid chunking
    key_pool = torch.zeros((rows // 16 + 1, layers, 16, 2, 64), dtype=torch.bfloat16, device=gpu)
    value_pool = torch.zeros_like(key_pool)
    gen = torch.Generator().manual_seed(4)
    slots = torch.randperm(key_pool.shape[0] * 16, generator=gen)[:rows]
    blocks, offsets = slots // 16, slots % 16
    k = pool((layers, rows, 2, 64), torch.bfloat16, gpu, 5)
    v = pool((layers, rows, 2, 64), torch.bfloat16, gpu, 6)
    kv_append_layers(key_pool, value_pool, 0, k, v, blocks.to(gpu), offsets.to(gpu))
    got_k = key_pool[blocks.to(gpu), :, offsets.to(gpu)]  # [rows, layers, H, D]
    assert torch.equal(got_k.transpose(0, 1), k)
    got_v = value_pool[blocks.to(gpu), :, offsets.to(gpu)]
    assert torch.equal(got_v.transpose(0, 1), v)


def test_append_skips_out_of_range_addresses(gpu):
    """A block id outside the pool or an offset outside the block writes
    nothing (the reference's index_put would raise; here the pool is never
    written outside its blocks), and every in-range row is still written,
    through both the Python adapter and the torch operator."""
    from vllm_rlt.kernels._extension import load_extension
    from vllm_rlt.kernels.hip_attention import kv_append

    load_extension()
    for via_op in (False, True):
        key_pool = pool((9, 2, 16, 4, 32), torch.bfloat16, gpu, 10)
        value_pool = pool((9, 2, 16, 4, 32), torch.bfloat16, gpu, 11)
        # a guard region after the pool: the layer view's last block is followed
        # by other memory of the same allocation
        kc, vc = key_pool[:8, 1], value_pool[:8, 1]
        before_k, before_v = key_pool.clone(), value_pool.clone()
        k = pool((5, 4, 32), torch.bfloat16, gpu, 12)
        v = pool((5, 4, 32), torch.bfloat16, gpu, 13)
        blocks = torch.tensor([0, 8, -1, 3, 7], dtype=torch.int64, device=gpu)
        offsets = torch.tensor([1, 0, 2, 16, 15], dtype=torch.int64, device=gpu)
        if via_op:
            torch.ops.vllm_rlt_hip.kv_append(kc, vc, k, v, blocks, offsets, None, None)
        else:
            kv_append(kc, vc, k, v, blocks, offsets)
        torch.cuda.synchronize()
        want_k, want_v = before_k.clone(), before_v.clone()
        for r in (0, 4):  # the two in-range rows
            want_k[blocks[r], 1, offsets[r]] = k[r]
            want_v[blocks[r], 1, offsets[r]] = v[r]
        assert torch.equal(key_pool, want_k) and torch.equal(value_pool, want_v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gather_is_bit_exact(gpu, dtype):
    from vllm_rlt.kernels.hip_attention import kv_gather

    key_pool = pool((50, 2, 16, 4, 32), dtype, gpu, 7)
    value_pool = pool((50, 2, 16, 4, 32), dtype, gpu, 8)
    table = torch.randperm(50, generator=torch.Generator().manual_seed(9))[:20].to(torch.int32)
    for length in (0, 1, 16, 17, 319, 320):
        keys, values = kv_gather(key_pool[:, 1], value_pool[:, 1], table.to(gpu), length)
        ek, ev = ref.kv_gather(as_np(key_pool[:, 1]), as_np(value_pool[:, 1]), table.numpy(),
                               length)
        assert np.array_equal(as_np(keys), ek) and np.array_equal(as_np(values), ev)


def test_finalize_rows_is_bit_exact(gpu):
    from vllm_rlt.kernels.hip_attention import kv_finalize

    slots, planes, width, layers = 5, 4, 6, 3
    n_blocks = slots * planes * width
    key_pool = pool((n_blocks, layers, 16, 2, 64), torch.bfloat16, gpu, 10)
    value_pool = pool((n_blocks, layers, 16, 2, 64), torch.bfloat16, gpu, 11)
    gen = torch.Generator().manual_seed(12)
    tables = torch.randperm(n_blocks, generator=gen).to(torch.int32).view(slots * planes, width)
    desc = torch.tensor([[0, 0, 5], [1, 2, 95], [3, 3, 40], [4, 1, 16], [2, 0, 0]],
                        dtype=torch.int64)
    ek, ev = as_np(key_pool), as_np(value_pool)
    ref.finalize_rows(ek, ev, desc.numpy(), tables.numpy(), planes)
    kv_finalize(key_pool, value_pool, desc.to(gpu), tables.to(gpu), planes)
    assert np.array_equal(as_np(key_pool), ek) and np.array_equal(as_np(value_pool), ev)


def test_finalize_token_is_bit_exact(gpu):
    from vllm_rlt.kernels.hip_attention import kv_finalize_token

    key_pool = pool((10, 5, 4, 3, 16), torch.float32, gpu, 13)
    value_pool = pool((10, 5, 4, 3, 16), torch.float32, gpu, 14)
    ek, ev = as_np(key_pool), as_np(value_pool)
    ref.finalize_token(ek, ev, 7, [2, 9], 3, [0, 2, 4])
    kv_finalize_token(key_pool, value_pool, 7, [2, 9], 3, [0, 2, 4])
    assert np.array_equal(as_np(key_pool), ek) and np.array_equal(as_np(value_pool), ev)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_copy_blocks_is_bit_exact(gpu, dtype):
    from vllm_rlt.kernels.hip_attention import kv_copy_blocks

    key_pool = pool((64, 3, 16, 4, 64), dtype, gpu, 15)
    value_pool = pool((64, 3, 16, 4, 64), dtype, gpu, 16)
    src = torch.tensor([0, 5, 63, 17], dtype=torch.int64)
    dst = torch.tensor([1, 40, 2, 18], dtype=torch.int64)
    ek, ev = as_np(key_pool), as_np(value_pool)
    ref.copy_blocks(ek, ev, src.numpy(), dst.numpy())
    kv_copy_blocks(key_pool, value_pool, src.to(gpu), dst.to(gpu))
    assert np.array_equal(as_np(key_pool), ek) and np.array_equal(as_np(value_pool), ev)


def test_expand_addresses_and_routing_are_exact(gpu):
    from vllm_rlt.kernels.hip_attention import (
        expand_kv_addresses,
        routing_metadata,
        routing_slots,
    )

    gen = torch.Generator().manual_seed(17)
    tables = torch.randint(0, 1000, (6, 9), generator=gen, dtype=torch.int32)
    positions = torch.randint(0, 9 * 16, (50,), generator=gen)
    sequences = torch.randint(0, 6, (50,), generator=gen, dtype=torch.int32)
    blocks, offsets = expand_kv_addresses(positions.to(gpu), sequences.to(gpu), tables.to(gpu),
                                          16)
    eb, eo = ref.expand_kv_addresses(positions.numpy(), sequences.numpy(), tables.numpy(), 16)
    assert np.array_equal(blocks.cpu().numpy(), eb) and np.array_equal(offsets.cpu().numpy(), eo)

    slots_n, planes, width, page = 4, 3, 7, 16
    route_tables = torch.randint(0, 500, (slots_n * planes, width), generator=gen,
                                 dtype=torch.int32)
    desc = torch.tensor([[2, 1, 30], [0, 2, 111], [3, 0, 0]], dtype=torch.int64)
    n, size, out_width = 3, 5, 4
    outs = dict(
        slots=torch.full((size,), -1, dtype=torch.int64, device=gpu),
        positions=torch.full((size,), -1, dtype=torch.int64, device=gpu),
        lengths=torch.full((size,), -1, dtype=torch.int32, device=gpu),
        blocks=torch.full((size,), -1, dtype=torch.int64, device=gpu),
        offsets=torch.full((size,), -1, dtype=torch.int64, device=gpu),
        out_tables=torch.full((size, width), -1, dtype=torch.int32, device=gpu),
    )
    routing_metadata(desc.to(gpu), route_tables.to(gpu), n=n, size=size, width=width, page=page,
                     planes=planes, out_width=out_width, **outs)
    expected = ref.routing_metadata(desc.numpy(), route_tables.numpy(), n, size, width, page,
                                    planes, out_width)
    for key, value in expected.items():
        assert np.array_equal(outs[key].cpu().numpy(), value), key
    slots = torch.full((size,), -1, dtype=torch.int64, device=gpu)
    routing_slots(desc.to(gpu), slots, n, size)
    assert np.array_equal(slots.cpu().numpy(), ref.routing_slots(desc.numpy(), n, size))
