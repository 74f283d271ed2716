"""Host side of the paged pool and the metadata builder on the CPU (no kernel
runs): write addresses and planned tables written out by hand, and the
argument checks that precede every device operation."""

import pytest
import torch

from vllm_rlt.core.paged_kv import PageSnapshot, PagedKVPool
from vllm_rlt.worker.metadata import build_kv_metadata, device_kv_metadata, write_addresses


def test_metadata_of_depth_selected_rows():
    # request a: planes [[3, 9, 4], [7, 1, 8], [0, 5, 6]]; request b: [[2, 10], ...]
    a = [[3, 9, 4], [7, 1, 8], [0, 5, 6]]
    b = [[2, 10]]
    rows = [a[2], b[0], a[1]]  # (a, depth 2, pos 4), (b, depth 0, pos 1), (a, depth 1, pos 2)
    batch = build_kv_metadata(rows, [4, 1, 2], block_size=2, device="cpu")
    assert batch.write_blocks.tolist() == [6, 2, 1]
    assert batch.write_offsets.tolist() == [0, 1, 0]
    assert batch.position_ids.tolist() == [4, 1, 2]
    assert batch.context_lengths.tolist() == [5, 2, 3]
    # padded to the batch width max(pos // bs + 1) = 3 with -1
    assert batch.block_tables.tolist() == [[0, 5, 6], [2, 10, -1], [7, 1, 8]]
    assert batch.write_blocks.dtype == torch.int64
    assert batch.block_tables.dtype == batch.context_lengths.dtype == torch.int32
    assert batch.cu_seqlens_q is None and batch.max_seqlen_q == 1


def test_packed_metadata_matches_the_reference_literal_case():
    """tests/test_flash_attention.py:121-143: positions [7, 8, 9] of one
    sequence and [3, 4] of another on 4-token pages."""
    a, b = [10, 11, 12, 13, 14], [20, 21, 22, 23, 24]
    batch = build_kv_metadata([a, a, a, b, b], [7, 8, 9, 3, 4], block_size=4, device="cpu",
                              sequence_keys=[("a", 0)] * 3 + [("b", 1)] * 2, packed=True,
                              for_write=True)
    assert batch.block_tables.shape == (2, 3)
    assert batch.context_lengths.tolist() == [10, 5]
    assert batch.cu_seqlens_q.tolist() == [0, 3, 5]
    assert batch.max_seqlen_q == 3
    assert batch.write_blocks.tolist() == [11, 12, 12, 20, 21]
    assert batch.write_offsets.tolist() == [3, 0, 1, 3, 0]
    with pytest.raises(ValueError, match="contiguous"):
        build_kv_metadata([a, a], [1, 3], block_size=4, device="cpu",
                          sequence_keys=[("a", 0)] * 2, packed=True)
    with pytest.raises(ValueError, match="one sequence"):
        build_kv_metadata([a, b, a], [1, 1, 2], block_size=4, device="cpu",
                          sequence_keys=[("a", 0), ("b", 0), ("a", 0)], packed=True)


def test_write_addresses_refuse_aliases_and_uncovered_positions():
    with pytest.raises(ValueError, match="duplicate"):
        write_addresses([[4, 5], [4, 6]], [1, 1], 2)
    assert write_addresses([[4, 5], [4, 6]], [1, 1], 2, for_write=False) == ([4, 4], [1, 1])
    with pytest.raises(ValueError, match="outside"):
        write_addresses([[4]], [2], 2)
    with pytest.raises(ValueError, match="equal lengths"):
        write_addresses([[4]], [0, 1], 2)


def test_device_metadata_checks():
    rows = 4
    ok = dict(position_ids=torch.arange(rows), write_blocks=torch.zeros(rows, dtype=torch.int64),
              write_offsets=torch.zeros(rows, dtype=torch.int64),
              block_tables=torch.zeros(rows, 2, dtype=torch.int32),
              context_lengths=torch.ones(rows, dtype=torch.int32))
    batch = device_kv_metadata(**ok, write_mask=torch.ones(rows, dtype=torch.bool),
                               active_rows=torch.tensor(3, dtype=torch.int32))
    assert batch.write_mask.dtype == torch.bool
    with pytest.raises(ValueError, match="write_mask"):
        device_kv_metadata(**ok, write_mask=torch.ones(rows, dtype=torch.int32))
    with pytest.raises(ValueError, match="active_rows"):
        device_kv_metadata(**ok, active_rows=torch.tensor([1, 2], dtype=torch.int32))
    with pytest.raises(ValueError, match="context_lengths"):
        device_kv_metadata(**{**ok, "context_lengths": torch.ones(rows, dtype=torch.int64)})
    with pytest.raises(ValueError, match="block tables"):
        device_kv_metadata(**{**ok, "block_tables": torch.zeros(rows, 0, dtype=torch.int32)})


def make_pool(**kwargs):
    parameters = dict(num_blocks=12, num_layers=2, block_size=2, num_kv_heads=1, head_dim=4,
                      dtype=torch.float32, device="cpu")
    parameters.update(kwargs)
    return PagedKVPool(**parameters)


def test_pool_shape_and_argument_checks():
    pool = make_pool()
    assert pool.key_cache.shape == (12, 2, 2, 1, 4) and not pool.key_cache.any()
    with pytest.raises(ValueError, match="num_blocks"):
        make_pool(num_blocks=0)
    with pytest.raises(ValueError, match="float32, float16 and bfloat16"):
        make_pool(dtype=torch.int8)
    with pytest.raises(ValueError, match="layer"):
        pool.layer(2)
    with pytest.raises(ValueError, match="out of range"):
        pool.copy_blocks([0], [99])
    with pytest.raises(ValueError, match="disjoint"):
        pool.copy_blocks([1, 2], [2, 3])
    with pytest.raises(ValueError, match="distinct"):
        pool.copy_blocks([1, 2], [3, 3])
    with pytest.raises(ValueError, match="equal lengths"):
        pool.copy_blocks([1], [])
    with pytest.raises(ValueError, match="exit_depth"):
        pool.finalize_token([[0], [1]], 0, 2)
    with pytest.raises(ValueError, match="beyond"):
        pool.finalize_token([[0], [1]], 2, 0)
    with pytest.raises(ValueError, match="length"):
        pool.read(0, [1], 3)
    snapshot = PageSnapshot(torch.zeros(2, 2, 2, 1, 4), torch.zeros(2, 2, 2, 1, 4))
    with pytest.raises(ValueError, match="page count"):
        pool.restore([1, 2, 3], snapshot)
    with pytest.raises(ValueError, match="distinct"):
        pool.restore([1, 1], snapshot)
    # nothing to copy: no kernel is reached
    pool.finalize_token([[0, 1]], 1, 0)
    pool.copy_blocks([], [])
