"""The reference's KV-cache flows, expressed directly on a page pool and page
lists and run through the hip kernels: LAST_EXITED propagation and early exit
(tests/test_kv_cache.py:38-77), SHARED single plane, mixed depth / request
batches against dense attention (tests/test_attention.py:33-60), packed prefill
through host metadata, sliding windows, masked and bucketed device writes
(kernels/graph_kv.py:7-65), snapshot / restore (tests/test_kv_cache.py:261-303)
and aliased prefix pages with a copy-on-write block copy. Checks are closed
forms, exact equality and torch's SDPA."""

import pytest
import torch
from torch.nn import functional as F

pytestmark = pytest.mark.gpu


def make_pool(**kwargs):
    from vllm_rlt.core.paged_kv import PagedKVPool

    parameters = dict(num_blocks=18, num_layers=2, block_size=2, num_kv_heads=1, head_dim=4,
                      dtype=torch.float32, device="cuda")
    parameters.update(kwargs)
    return PagedKVPool(**parameters)


def full(shape, value, dtype=torch.float32):
    return torch.full(shape, float(value), device="cuda", dtype=dtype)


def write(pool, layer, pages_per_row, positions, k, v):
    """Append rows through host-built metadata (the manager's write path)."""
    from vllm_rlt.worker.metadata import build_kv_metadata

    batch = build_kv_metadata(pages_per_row, positions, block_size=pool.block_size,
                              device=pool.device)
    pool.append(layer, k, v, batch.write_blocks, batch.write_offsets)
    return batch


def attend(pool, layer, pages_per_row, positions, q, window=None):
    from vllm_rlt.worker.metadata import build_kv_metadata

    batch = build_kv_metadata(pages_per_row, positions, block_size=pool.block_size,
                              device=pool.device, for_write=False)
    return pool.attend(layer, q, batch.block_tables, batch.context_lengths, window=window)


def dense_attention(q, k, v):
    groups = q.shape[0] // k.shape[1]
    return F.scaled_dot_product_attention(
        q.float()[None, :, None],
        k.float().repeat_interleave(groups, dim=1).transpose(0, 1)[None],
        v.float().repeat_interleave(groups, dim=1).transpose(0, 1)[None],
    )[0, :, 0].to(q.dtype)


PLANES = [[4, 11], [1, 7], [3, 9]]  # one request, 3 depth planes of 2 pages


def test_last_exited_copies_every_layer_and_preserves_executed_depths(gpu):
    pool = make_pool()
    for layer in range(2):
        for depth in range(2):
            keys = full((1, 1, 4), 10 * layer + depth)
            write(pool, layer, [PLANES[depth]], [0], keys, keys + 100)
    pool.finalize_token(PLANES, 0, exit_depth=1)
    for layer in range(2):
        first_keys, first_values = pool.read(layer, PLANES[0], 1)
        second_keys, second_values = pool.read(layer, PLANES[1], 1)
        last_keys, last_values = pool.read(layer, PLANES[2], 1)
        assert torch.equal(first_keys, full((1, 1, 4), 10 * layer))
        assert torch.equal(first_values, full((1, 1, 4), 10 * layer + 100))
        assert torch.equal(last_keys, second_keys) and torch.equal(last_values, second_values)
    # physical copies: a later write at depth 1 does not reach depth 2
    write(pool, 0, [PLANES[1]], [0], full((1, 1, 4), 0), full((1, 1, 4), 0))
    assert torch.equal(pool.read(0, PLANES[2], 1)[0], full((1, 1, 4), 1))


def test_early_exit_then_deeper_token_across_page_boundary(gpu):
    pool = make_pool()
    for position, exit_depth in [(0, 0), (1, 1), (2, 2)]:
        for depth in range(exit_depth + 1):
            for layer in range(2):
                keys = full((1, 1, 4), position * 10 + depth + layer)
                write(pool, layer, [PLANES[depth]], [position], keys, keys + 100)
                attended = attend(pool, layer, [PLANES[depth]], [position],
                                  torch.zeros(1, 2, 4, device="cuda"))
                expected = torch.tensor(
                    [100 + p * 10 + min(p, depth) + layer for p in range(position + 1)]
                ).float().mean()
                torch.testing.assert_close(attended.cpu(), torch.full((1, 2, 4), float(expected)))
        pool.finalize_token(PLANES, position, exit_depth)
    assert pool.read(0, PLANES[2], 3)[0].shape == (3, 1, 4)


def test_shared_layout_single_plane(gpu):
    pool = make_pool()
    shared = [[5, 2]]  # every depth reads and writes the one plane
    for depth in range(3):
        write(pool, 1, shared, [depth], full((1, 1, 4), depth), full((1, 1, 4), depth))
    keys, _ = pool.read(1, shared[0], 3)
    assert torch.equal(keys[:, 0, 0].cpu(), torch.tensor([0.0, 1.0, 2.0]))
    before = pool.key_cache.clone()
    pool.finalize_token(shared, 0, 0)  # no deeper plane: nothing is copied
    torch.cuda.synchronize()
    assert torch.equal(pool.key_cache, before)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [7, 32, 64, 128])
def test_mixed_depth_and_request_batch_matches_dense(gpu, dtype, head_dim):
    """tests/test_attention.py:33-60: rows of two requests at different depths
    and positions in one call, on 3-token pages."""
    torch.manual_seed(48)
    pool = make_pool(num_blocks=48, num_kv_heads=2, head_dim=head_dim, block_size=3, dtype=dtype)
    order = torch.randperm(48, generator=torch.Generator().manual_seed(1)).tolist()
    planes = {("a", d): order[3 * d : 3 * d + 3] for d in range(3)}
    planes.update({("b", d): order[9 + 2 * d : 11 + 2 * d] for d in range(3)})
    histories = {}
    for request, length in [("a", 7), ("b", 6)]:
        for depth in range(3):
            k = torch.randn(length, 2, head_dim, device="cuda", dtype=dtype) + depth * 0.5
            v = torch.randn_like(k) + (4 if request == "a" else -4)
            write(pool, 1, [planes[request, depth]] * length, list(range(length)), k, v)
            histories[request, depth] = k, v
    rows = [("a", 2, 6), ("b", 0, 4), ("a", 1, 2), ("b", 2, 5)]
    q = torch.randn(4, 6, head_dim, device="cuda", dtype=dtype)
    actual = attend(pool, 1, [planes[r, d] for r, d, _ in rows], [p for *_, p in rows], q)
    expected = torch.stack([dense_attention(q[i], *(t[: p + 1] for t in histories[r, d]))
                            for i, (r, d, p) in enumerate(rows)])
    tol = 2e-2 if dtype == torch.bfloat16 else 2e-3 if dtype == torch.float16 else 2e-5
    torch.testing.assert_close(actual, expected, atol=tol, rtol=tol)


def test_packed_prefill_through_host_metadata(gpu):
    """Packed rows (one 70-query chunk and one decode row) equal per-row
    single-query attention over the same pages."""
    from vllm_rlt.worker.metadata import build_kv_metadata

    torch.manual_seed(7)
    pool = make_pool(num_layers=1, num_kv_heads=2, head_dim=64, num_blocks=64, block_size=16,
                     dtype=torch.bfloat16)
    a, b = list(range(10, 20)), [40, 41, 42]
    ka = torch.randn(150, 2, 64, device="cuda", dtype=torch.bfloat16)
    kb = torch.randn(40, 2, 64, device="cuda", dtype=torch.bfloat16)
    write(pool, 0, [a] * 150, list(range(150)), ka, ka * 0.5)
    write(pool, 0, [b] * 40, list(range(40)), kb, kb * 0.5)
    rows = [a] * 70 + [b]
    positions = list(range(80, 150)) + [39]
    batch = build_kv_metadata(rows, positions, block_size=16, device="cuda",
                              sequence_keys=[("a", 1)] * 70 + [("b", 0)], packed=True,
                              for_write=False)
    assert batch.cu_seqlens_q.tolist() == [0, 70, 71]
    q = torch.randn(71, 4, 64, device="cuda", dtype=torch.bfloat16)
    packed = pool.prefill(0, q, batch.block_tables, batch.context_lengths, batch.cu_seqlens_q,
                          batch.max_seqlen_q)
    single = attend(pool, 0, rows, positions, q)
    torch.testing.assert_close(packed.float(), single.float(), atol=2e-2, rtol=2e-2)


def test_windowed_attend_matches_sliced_dense(gpu):
    torch.manual_seed(9)
    pool = make_pool(num_layers=1, head_dim=32, num_blocks=40, block_size=4)
    pages = list(range(39, 24, -1))
    k = torch.randn(60, 1, 32, device="cuda")
    v = torch.randn(60, 1, 32, device="cuda")
    write(pool, 0, [pages] * 60, list(range(60)), k, v)
    q = torch.randn(3, 2, 32, device="cuda")
    positions = [5, 30, 59]
    out = attend(pool, 0, [pages] * 3, positions, q, window=8)
    expected = torch.stack([dense_attention(q[i], k[max(0, p - 7) : p + 1],
                                            v[max(0, p - 7) : p + 1])
                            for i, p in enumerate(positions)])
    torch.testing.assert_close(out, expected, atol=2e-5, rtol=2e-5)


def test_device_metadata_masked_and_bucketed_writes(gpu):
    """write_mask and active_rows skip rows (kernels/graph_kv.py semantics)."""
    from vllm_rlt.worker.metadata import device_kv_metadata

    pool = make_pool(num_layers=1, num_blocks=12)
    pages = [6, 2, 9, 4]
    positions = torch.tensor([0, 1, 2, 3], device="cuda")
    blocks = torch.tensor([pages[p // 2] for p in range(4)], device="cuda")
    offsets = positions % 2
    batch = device_kv_metadata(
        position_ids=positions, write_blocks=blocks, write_offsets=offsets,
        block_tables=torch.tensor([pages] * 4, dtype=torch.int32, device="cuda"),
        context_lengths=(positions + 1).to(torch.int32),
        write_mask=torch.tensor([True, False, True, True], device="cuda"),
        active_rows=torch.tensor(3, dtype=torch.int32, device="cuda"))
    k = torch.arange(1, 5, dtype=torch.float32, device="cuda").view(4, 1, 1).expand(4, 1, 4)
    pool.append(0, k.contiguous(), k.contiguous(), batch.write_blocks, batch.write_offsets,
                write_mask=batch.write_mask, active_rows=batch.active_rows)
    written = pool.key_cache[blocks, 0, offsets][:, 0, 0].cpu().tolist()
    assert written == [1.0, 0.0, 3.0, 0.0]


def test_snapshot_restore_round_trip(gpu):
    """tests/test_kv_cache.py:261-303: every page of every plane to host, a
    disturbed pool, restore into other pages, byte-equal reads; a target with
    another page count is refused."""
    pool = make_pool(num_blocks=12)
    for depth in (0, 1):
        for layer in range(2):
            for position in (0, 1):
                k = full((1, 1, 4), 2 + depth + 10 * layer + position)
                write(pool, layer, [PLANES[depth]], [position], k, -k)
    pool.finalize_token(PLANES, 0, 1)
    before = {(d, layer): pool.read(layer, PLANES[d], 2) for d in range(3) for layer in range(2)}
    pages = [p for plane in PLANES for p in plane]
    snapshot = pool.snapshot(pages)
    assert snapshot.pages == 6 and snapshot.keys.is_pinned()
    pool.key_cache.fill_(-1.0)
    pool.value_cache.fill_(-1.0)
    moved = [[0, 2], [5, 6], [8, 10]]
    with pytest.raises(ValueError, match="page count"):
        pool.restore([0, 2, 5, 6], snapshot)
    pool.restore([p for plane in moved for p in plane], snapshot)
    for (d, layer), (keys, values) in before.items():
        got_k, got_v = pool.read(layer, moved[d], 2)
        assert torch.equal(got_k, keys) and torch.equal(got_v, values)


def test_aliased_prefix_pages_and_copy_on_write(gpu):
    """Two requests alias one prefix page (zero-copy sharing); a divergent
    write first copies the page to a private block; the other request keeps
    reading the original bytes."""
    pool = make_pool(num_layers=2, num_blocks=30)
    a = [3, 8, 12]
    for layer in range(2):
        for p in range(4):
            write(pool, layer, [a], [p], full((1, 1, 4), p), full((1, 1, 4), -p))
    b = [3, 8, 20]  # shares a's first two pages
    keys, _ = pool.read(1, b, 4)
    assert keys[:, 0, 0].cpu().tolist() == [0.0, 1.0, 2.0, 3.0]
    pool.copy_blocks([8], [21])
    torch.cuda.synchronize()
    assert torch.equal(pool.key_cache[21], pool.key_cache[8])
    assert torch.equal(pool.value_cache[21], pool.value_cache[8])
    b = [3, 21, 20]
    write(pool, 0, [b], [3], full((1, 1, 4), 99), full((1, 1, 4), 99))
    assert pool.read(0, b, 4)[0][:, 0, 0].cpu().tolist() == [0.0, 1.0, 2.0, 99.0]
    assert pool.read(0, a, 4)[0][:, 0, 0].cpu().tolist() == [0.0, 1.0, 2.0, 3.0]
    with pytest.raises(ValueError, match="disjoint"):
        pool.copy_blocks([8], [8])
