"""The KV manager mirror on the GPU: the reference's own flows
(tests/test_kv_cache.py, tests/test_attention.py:18-132, tests/test_prepared_kv.py)
run through the hip kernels, checked with closed forms, exact equality and an
independent SDPA oracle."""

import pytest
import torch
from torch.nn import functional as F

pytestmark = pytest.mark.gpu


def make_cache(**kwargs):
    from vllm_rlt.core.kv_cache_manager import KVCacheManager

    parameters = dict(num_layers=2, num_kv_heads=1, head_dim=4, num_blocks=18, block_size=2,
                      max_loops=3, device="cuda", dtype=torch.float32, backend="hip")
    parameters.update(kwargs)
    return KVCacheManager(**parameters)


def dense_attention(q, k, v):
    groups = q.shape[0] // k.shape[1]
    return F.scaled_dot_product_attention(
        q.float()[None, :, None],
        k.float().repeat_interleave(groups, dim=1).transpose(0, 1)[None],
        v.float().repeat_interleave(groups, dim=1).transpose(0, 1)[None],
    )[0, :, 0].to(q.dtype)


def full(shape, value):
    return torch.full(shape, float(value), device="cuda")


def test_backend_is_hip(gpu):
    cache = make_cache()
    assert cache.backend == "hip"
    assert cache.attention_capabilities.packed_prefill


def test_last_exited_copies_every_layer_and_preserves_executed_depths(gpu):
    cache = make_cache()
    assert cache.allocate("a", 4)
    for layer in range(2):
        for depth in range(2):
            keys = full((1, 1, 4), 10 * layer + depth)
            cache.write(layer, ["a"], [depth], [0], keys, keys + 100)
    cache.finalize_token("a", 0, exit_depth=1)
    for layer in range(2):
        first_keys, first_values = cache.read(layer, "a", 0, 1)
        second_keys, second_values = cache.read(layer, "a", 1, 1)
        last_keys, last_values = cache.read(layer, "a", 2, 1)
        assert torch.equal(first_keys, full((1, 1, 4), 10 * layer))
        assert torch.equal(first_values, full((1, 1, 4), 10 * layer + 100))
        assert torch.equal(last_keys, second_keys) and torch.equal(last_values, second_values)
    cache.write(0, ["a"], [1], [0], full((1, 1, 4), 0), full((1, 1, 4), 0))
    assert torch.equal(cache.read(0, "a", 2, 1)[0], full((1, 1, 4), 1))


def test_early_exit_then_deeper_token_across_block_boundary(gpu):
    cache = make_cache()
    assert cache.allocate("a", 3)
    for position, exit_depth in [(0, 0), (1, 1), (2, 2)]:
        for depth in range(exit_depth + 1):
            for layer in range(2):
                keys = full((1, 1, 4), position * 10 + depth + layer)
                cache.write(layer, ["a"], [depth], [position], keys, keys + 100)
                attended = cache.attend(layer, ["a"], [depth], [position],
                                        torch.zeros(1, 2, 4, device="cuda"))
                expected = torch.tensor(
                    [100 + p * 10 + min(p, depth) + layer for p in range(position + 1)]
                ).float().mean()
                torch.testing.assert_close(attended.cpu(), torch.full((1, 2, 4), float(expected)))
        cache.finalize_token("a", position, exit_depth)
    assert cache.read(0, "a", 2)[0].shape == (3, 1, 4)


def test_block_reuse_never_exposes_stale_history(gpu):
    cache = make_cache(num_blocks=6)
    assert cache.allocate("old", 4)
    cache.write(0, ["old"] * 4, [0] * 4, list(range(4)), full((4, 1, 4), 7), full((4, 1, 4), 7))
    cache.free("old")
    assert cache.allocate("new", 4)
    with pytest.raises(RuntimeError, match="uninitialized"):
        cache.attend(0, ["new"], [0], [0], full((1, 1, 4), 1))
    cache.write(0, ["new"], [0], [0], full((1, 1, 4), 0), full((1, 1, 4), 1))
    assert torch.equal(cache.attend(0, ["new"], [0], [0], full((1, 1, 4), 0)), full((1, 1, 4), 1))


def test_validation_happens_before_mutation(gpu):
    cache = make_cache()
    cache.allocate("a", 3)
    k = full((2, 1, 4), 1)
    with pytest.raises(ValueError, match="position"):
        cache.write(0, ["a", "a"], [0, 0], [0, 3], k, k)
    assert cache.read(0, "a", 0)[0].shape[0] == 0
    with pytest.raises(ValueError, match="duplicate"):
        cache.write(0, ["a", "a"], [0, 0], [0, 0], k, k)
    with pytest.raises(RuntimeError, match="every layer"):
        cache.finalize_token("a", 0, 0)
    with pytest.raises(ValueError, match="dtype"):
        cache.write(0, ["a"], [0], [0], k[:1].half(), k[:1].half())


def test_out_of_order_writes_only_expose_complete_prefix(gpu):
    cache = make_cache()
    cache.allocate("a", 4)
    k = torch.arange(16, dtype=torch.float32, device="cuda").reshape(4, 1, 4)
    cache.write(0, ["a", "a"], [0, 0], [3, 1], k[[3, 1]], k[[3, 1]])
    assert cache.read(0, "a", 0)[0].shape[0] == 0
    cache.write(0, ["a"], [0], [0], k[:1], k[:1])
    assert torch.equal(cache.read(0, "a", 0)[0], k[:2])
    with pytest.raises(RuntimeError, match="uninitialized"):
        cache.attend(0, ["a"], [0], [3], torch.zeros(1, 1, 4, device="cuda"))
    cache.write(0, ["a"], [0], [2], k[2:3], k[2:3])
    assert torch.equal(cache.read(0, "a", 0)[0], k)


def test_shared_layout_single_plane(gpu):
    cache = make_cache(layout="shared")
    assert cache.allocate("a", 4)
    assert len(cache.plane_block_tables("a")) == 1
    for depth in range(3):
        cache.write(1, ["a"], [depth], [depth], full((1, 1, 4), depth), full((1, 1, 4), depth))
    keys, _ = cache.read(1, "a", 2)
    assert torch.equal(keys[:, 0, 0].cpu(), torch.tensor([0.0, 1.0, 2.0]))
    cache.write(0, ["a"], [0], [0], full((1, 1, 4), 5), full((1, 1, 4), 5))
    cache.finalize_token("a", 0, 0)  # no copies under SHARED
    assert torch.equal(cache.read(0, "a", 2, 1)[0], full((1, 1, 4), 5))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [7, 32, 64, 128])
def test_mixed_depth_and_request_batch_matches_dense(gpu, dtype, head_dim):
    """tests/test_attention.py:33-60 on the hip backend."""
    torch.manual_seed(48)
    cache = make_cache(num_layers=2, num_kv_heads=2, head_dim=head_dim, num_blocks=48,
                       block_size=3, max_loops=3, dtype=dtype)
    cache.allocate("retained", 4)
    cache.allocate("hole", 8)
    cache.allocate("a", 7)
    cache.free("hole")
    cache.allocate("b", 6)
    histories = {}
    for request_id, length in [("a", 7), ("b", 6)]:
        for depth in range(3):
            k = torch.randn(length, 2, head_dim, device="cuda", dtype=dtype) + depth * 0.5
            v = torch.randn_like(k) + (4 if request_id == "a" else -4)
            cache.write(1, [request_id] * length, [depth] * length, list(range(length)), k, v)
            histories[request_id, depth] = k, v
    request_ids, depths, positions = ["a", "b", "a", "b"], [2, 0, 1, 2], [6, 4, 2, 5]
    q = torch.randn(4, 6, head_dim, device="cuda", dtype=dtype)
    actual = cache.attend(1, request_ids, depths, positions, q)
    expected = torch.stack([
        dense_attention(q[row], *(t[: p + 1] for t in histories[r, d]))
        for row, (r, d, p) in enumerate(zip(request_ids, depths, positions))
    ])
    tol = 2e-2 if dtype == torch.bfloat16 else 2e-3 if dtype == torch.float16 else 2e-5
    torch.testing.assert_close(actual, expected, atol=tol, rtol=tol)


def test_packed_prefill_through_prepared_metadata(gpu):
    """Packed rows (prepare(packed=True)) equal per-row causal attention."""
    torch.manual_seed(7)
    cache = make_cache(num_layers=1, num_kv_heads=2, head_dim=64, num_blocks=64, block_size=16,
                       max_loops=2, dtype=torch.bfloat16)
    cache.allocate("a", 150)
    cache.allocate("b", 40)
    ka = torch.randn(150, 2, 64, device="cuda", dtype=torch.bfloat16)
    kb = torch.randn(40, 2, 64, device="cuda", dtype=torch.bfloat16)
    cache.write(0, ["a"] * 150, [1] * 150, list(range(150)), ka, ka * 0.5)
    cache.write(0, ["b"] * 40, [0] * 40, list(range(40)), kb, kb * 0.5)
    ids = ["a"] * 70 + ["b"] * 1
    depths = [1] * 70 + [0]
    positions = list(range(80, 150)) + [39]
    batch = cache.prepare(ids, depths, positions, packed=True, for_write=False)
    assert batch.cu_seqlens_q.tolist() == [0, 70, 71]
    q = torch.randn(71, 4, 64, device="cuda", dtype=torch.bfloat16)
    packed = cache._attend_prepared(0, batch, q)
    single = cache.attend(0, ids, depths, positions, q)
    torch.testing.assert_close(packed.float(), single.float(), atol=2e-2, rtol=2e-2)


def test_windowed_attend_matches_sliced_dense(gpu):
    torch.manual_seed(9)
    cache = make_cache(num_layers=1, num_kv_heads=1, head_dim=32, num_blocks=40, block_size=4,
                       max_loops=1)
    cache.allocate("a", 60)
    k = torch.randn(60, 1, 32, device="cuda")
    v = torch.randn(60, 1, 32, device="cuda")
    cache.write(0, ["a"] * 60, [0] * 60, list(range(60)), k, v)
    q = torch.randn(3, 2, 32, device="cuda")
    positions = [5, 30, 59]
    out = cache.attend(0, ["a"] * 3, [0] * 3, positions, q, window=8)
    expected = torch.stack([dense_attention(q[i], k[max(0, p - 7) : p + 1], v[max(0, p - 7) : p + 1])
                            for i, p in enumerate(positions)])
    torch.testing.assert_close(out, expected, atol=2e-5, rtol=2e-5)


def test_device_metadata_masked_and_bucketed_writes(gpu):
    """DeviceKVMetadata path: write_mask and active_rows skip rows (graph_kv semantics)."""
    cache = make_cache(num_layers=1, num_blocks=12)
    cache.allocate("a", 8)
    table = cache.get_block_table("a", 0)
    positions = torch.tensor([0, 1, 2, 3], device="cuda")
    blocks = torch.tensor([table[p // 2] for p in range(4)], device="cuda")
    offsets = positions % 2
    tables = torch.tensor([list(table)] * 4, dtype=torch.int32, device="cuda")
    lengths = (positions + 1).to(torch.int32)
    mask = torch.tensor([True, False, True, True], device="cuda")
    active = torch.tensor(3, dtype=torch.int32, device="cuda")
    batch = cache.metadata_builder.prepare_device(
        allocations=[("a", cache._allocations["a"])], position_ids=positions,
        write_blocks=blocks, write_offsets=offsets, block_tables=tables,
        context_lengths=lengths, write_mask=mask, active_rows=active)
    cache.key_cache.zero_()
    k = torch.arange(1, 5, dtype=torch.float32, device="cuda").view(4, 1, 1).expand(4, 1, 4)
    cache._write_prepared(0, batch, k.contiguous(), k.contiguous())
    written = cache.key_cache[blocks, 0, offsets][:, 0, 0].cpu().tolist()
    assert written == [1.0, 0.0, 3.0, 0.0]


def test_snapshot_restore_round_trip(gpu):
    from vllm_rlt.core.kv_cache_manager import KVSnapshot

    cache = make_cache(num_blocks=12)
    assert cache.allocate("a", 4)
    for depth in (0, 1):
        for layer in range(2):
            for position in (0, 1):
                k = full((1, 1, 4), 2 + depth + 10 * layer + position)
                cache.write(layer, ["a"], [depth], [position], k, -k)
    cache.finalize_token("a", 0, 1)
    before = {(d, layer): cache.read(layer, "a", d) for d in range(3) for layer in range(2)}
    snapshot = cache.snapshot("a")
    assert snapshot.pages == 2 and snapshot.keys.shape[0] == 6
    cache.free("a")
    assert cache.allocate("filler", 2)
    assert cache.allocate("a", 4)
    with pytest.raises(ValueError, match="page count"):
        cache.restore("a", KVSnapshot(4, 1, snapshot.written, snapshot.keys, snapshot.values))
    cache.restore("a", snapshot)
    torch.cuda.synchronize()
    for (d, layer), (keys, values) in before.items():
        got_k, got_v = cache.read(layer, "a", d)
        assert torch.equal(got_k, keys) and torch.equal(got_v, values)


def test_copy_blocks_and_prefix_sharing(gpu):
    """Refcounted prefix pages are aliased (zero-copy); copy_blocks makes a private copy."""
    cache = make_cache(num_layers=2, num_blocks=30, block_size=2, max_loops=2,
                       enable_prefix_caching=True)
    tokens = [5, 6, 7, 8, 9]
    assert cache.allocate("a", 6)
    for depth in range(2):
        for layer in range(2):
            for p in range(4):
                cache.write(layer, ["a"], [depth], [p], full((1, 1, 4), p), full((1, 1, 4), -p))
    cache.publish_prefix("a", tokens, 5)
    prefix = cache.lookup_prefix(tokens)
    assert len(prefix) == 2
    assert cache.allocate("b", 6, prefix=prefix)
    assert cache.get_block_table("b", 0)[:2] == cache.get_block_table("a", 0)[:2]
    keys, _ = cache.read(1, "b", 1, 4)
    assert keys[:, 0, 0].cpu().tolist() == [0.0, 1.0, 2.0, 3.0]
    shared = cache.get_block_table("b", 0)[1]
    spare = cache.get_block_table("b", 0)[2]
    cache.copy_blocks([shared], [spare])
    torch.cuda.synchronize()
    assert torch.equal(cache.key_cache[spare], cache.key_cache[shared])
    assert torch.equal(cache.value_cache[spare], cache.value_cache[shared])
    with pytest.raises(ValueError, match="disjoint"):
        cache.copy_blocks([shared], [shared])
