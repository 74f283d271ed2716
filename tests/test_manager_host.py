"""Host bookkeeping of the KV manager mirror on the CPU (no kernels run):
allocation atomicity, planes, prefix refcounts, metadata planning and the
validation that precedes any device work. Mirrors tests/test_kv_cache.py:15-358
and tests/test_prepared_kv.py of the reference."""

import pytest
import torch

from vllm_rlt.attention import AttentionBackend, BackendCapabilities
from vllm_rlt.core.kv_cache_manager import KVCacheManager


class _NoKernels:
    def __call__(self, *args):
        raise AssertionError("host-only test reached a kernel")

    prefill = windowed = __call__


def make_cache(**kwargs):
    parameters = dict(num_layers=2, num_kv_heads=1, head_dim=4, num_blocks=18, block_size=2,
                      max_loops=3, device="cpu", dtype=torch.float32)
    parameters.update(kwargs)
    caps = BackendCapabilities(packed_prefill=True)
    return KVCacheManager(**parameters,
                          attention=AttentionBackend(_NoKernels(), caps, {"backend": "stub"}))


def test_admission_is_atomic_and_counts_all_depths():
    cache = make_cache(num_blocks=12)
    assert cache.required_blocks(3) == 6
    assert cache.allocate("a", 3)
    assert cache.num_used_blocks == 6
    assert not cache.allocate("b", 5)
    assert cache.num_used_blocks == 6
    with pytest.raises(ValueError, match="pool has"):
        cache.allocate("impossible", 9)
    with pytest.raises(ValueError, match="already owns"):
        cache.allocate("a", 3)
    assert cache.allocate("b", 4)
    assert cache.num_free_blocks == 0
    cache.free("never-admitted")
    cache.free("a")
    cache.free("a")
    assert cache.num_free_blocks == 6
    assert cache.allocate("c", 4)
    c_pages = {p for d in range(3) for p in cache.get_block_table("c", d)}
    b_pages = {p for d in range(3) for p in cache.get_block_table("b", d)}
    assert c_pages.isdisjoint(b_pages)


def test_shared_layout_exposes_one_plane():
    cache = make_cache(layout="shared")
    assert cache.allocate("a", 4)
    assert len(cache.plane_block_tables("a")) == 1
    assert cache.allocated_blocks("a") == 2
    assert cache.get_block_table("a", 2) == cache.plane_block_tables("a")[0]
    with pytest.raises(ValueError, match="prefix caching requires"):
        make_cache(layout="shared", enable_prefix_caching=True)


def test_prefix_refcounts_and_exclusive_blocks():
    cache = make_cache(num_blocks=18, enable_prefix_caching=True)
    tokens = list(range(1, 6))
    assert cache.allocate("a", 6)
    cache.publish_prefix("a", tokens, 5)
    prefix = cache.lookup_prefix(tokens)
    assert len(prefix) == 2
    assert cache.exclusive_prefix_blocks(prefix) == 0
    cache.free("a")
    assert cache.exclusive_prefix_blocks(prefix) == 6
    assert cache.allocate("b", 6, prefix=prefix)
    assert cache.exclusive_prefix_blocks(prefix) == 0
    assert cache.get_block_table("b", 1)[:2] == tuple(g[1] for g in prefix)
    assert cache.prefix_hits == 4
    cache.free("b")
    assert cache.allocate("c", 2, prefix=prefix[:1])
    assert cache.exclusive_prefix_blocks(prefix) == 3


def test_validation_before_any_kernel():
    cache = make_cache()
    cache.allocate("a", 3)
    k = torch.ones(2, 1, 4)
    with pytest.raises(ValueError, match="position"):
        cache.write(0, ["a", "a"], [0, 0], [0, 3], k, k)
    with pytest.raises(ValueError, match="duplicate"):
        cache.write(0, ["a", "a"], [0, 0], [0, 0], k, k)
    with pytest.raises(ValueError, match="one-dimensional integer"):
        cache.write(0, ["a"], [0], torch.tensor([0.5]), k[:1], k[:1])
    with pytest.raises(ValueError, match="depth"):
        cache.get_block_table("a", 3)
    with pytest.raises(ValueError, match="dtype"):
        cache.write(0, ["a"], [0], [0], k[:1].half(), k[:1].half())
    with pytest.raises(RuntimeError, match="uninitialized"):
        cache.attend(0, ["a"], [0], [0], torch.zeros(1, 1, 4))
    with pytest.raises(ValueError, match="positive multiple"):
        cache.attend(0, ["a"], [0], [0], torch.zeros(1, 0, 4))
    with pytest.raises(KeyError, match="no KV allocation"):
        cache.read(0, "zzz", 0)
    with pytest.raises(ValueError, match="layer"):
        cache.write(2, ["a"], [0], [0], k[:1], k[:1])


def test_prepared_metadata_is_depth_selected_and_typed():
    cache = make_cache(block_size=2, max_loops=3)
    cache.allocate("a", 5)
    cache.allocate("b", 3)
    batch = cache.prepare(["a", "b", "a"], [2, 0, 1], [4, 1, 2], for_write=True)
    ta, tb = cache.plane_block_tables("a"), cache.plane_block_tables("b")
    assert batch.write_blocks.tolist() == [ta[2][2], tb[0][0], ta[1][1]]
    assert batch.write_offsets.tolist() == [0, 1, 0]
    assert batch.context_lengths.tolist() == [5, 2, 3]
    # rows keep their table up to the batch width (reference attention/metadata.py:86-90)
    assert batch.block_tables.tolist() == [list(ta[2][:3]), list(tb[0][:2]) + [-1],
                                           list(ta[1][:3])]
    assert batch.write_blocks.dtype == torch.int64
    assert batch.block_tables.dtype == batch.context_lengths.dtype == torch.int32
    packed = cache.prepare(["a", "a", "b"], [0, 0, 0], [1, 2, 0], packed=True, for_write=False)
    assert packed.cu_seqlens_q.tolist() == [0, 2, 3]
    assert packed.context_lengths.tolist() == [3, 1]
    assert packed.max_seqlen_q == 2


def test_stale_prepared_batch_is_rejected():
    cache = make_cache()
    cache.allocate("a", 3)
    batch = cache.prepare(["a"], [0], [0])
    cache.free("a")
    cache.allocate("a", 3)
    with pytest.raises(RuntimeError, match="stale"):
        cache._write_prepared(0, batch, torch.ones(1, 1, 4), torch.ones(1, 1, 4))


def test_copy_blocks_validation():
    cache = make_cache()
    with pytest.raises(ValueError, match="out of range"):
        cache.copy_blocks([0], [99])
    with pytest.raises(ValueError, match="disjoint"):
        cache.copy_blocks([1, 2], [2, 3])
    with pytest.raises(ValueError, match="equal lengths"):
        cache.copy_blocks([1], [])
