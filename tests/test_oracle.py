"""Pins the CPU oracle itself (CPU only).

Each check can fail for a plausible mistake in the oracle (wrong scale, GQA
head mapping, off-by-one window or causal length, dropped rows):
  * attention == torch.nn.functional.scaled_dot_product_attention (independent
    library routine; the reference pins its Torch path the same way,
    tests/test_attention.py:8-15,203-255);
  * closed forms: length 0 -> zeros, length 1 -> V row, constant keys -> mean V,
    window == slicing the history, the closed-form early-exit means of
    tests/test_kv_cache.py:61-77;
  * the committed golden fixture (tests/golden/decode_small.npz);
  * integer kernels against brute-force loops / literal vectors, including the
    packed-address vectors of tests/test_flash_attention.py:121-143;
  * finalize_token and the snapshot copies against the closed forms of
    tests/test_kv_cache.py:38-58 and :261-303.
"""

import math
import os

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from oracle import paged_ref as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def sdpa_rows(q, keys_per_row, values_per_row, groups):
    out = []
    for row in range(q.shape[0]):
        k = torch.from_numpy(keys_per_row[row]).repeat_interleave(groups, dim=1)
        v = torch.from_numpy(values_per_row[row]).repeat_interleave(groups, dim=1)
        if k.shape[0] == 0:
            out.append(torch.zeros(q.shape[1], q.shape[2]))
            continue
        o = F.scaled_dot_product_attention(
            torch.from_numpy(q[row])[:, None], k.transpose(0, 1), v.transpose(0, 1)
        )
        out.append(o[:, 0])
    return torch.stack(out).numpy()


def random_case(rng, lengths, heads=4, kv_heads=2, dim=16, block=4):
    pages = sum(-(-n // block) for n in lengths) + 2
    kc = rng.standard_normal((pages, block, kv_heads, dim)).astype(np.float32)
    vc = rng.standard_normal((pages, block, kv_heads, dim)).astype(np.float32)
    order = list(rng.permutation(pages))
    width = max(1, max(-(-n // block) for n in lengths))
    tables = np.full((len(lengths), width), -1, np.int32)
    for row, n in enumerate(lengths):
        for p in range(-(-n // block)):
            tables[row, p] = order.pop()
    q = rng.standard_normal((len(lengths), heads, dim)).astype(np.float32)
    return q, kc, vc, tables, np.asarray(lengths, np.int32)


def history(kc, tables, lengths, start=None):
    block = kc.shape[1]
    out = []
    for row, n in enumerate(lengths):
        s = 0 if start is None else start[row]
        pos = np.arange(s, n)
        out.append(kc[tables[row][pos // block], pos % block])
    return out


def test_attention_matches_sdpa_with_gqa():
    rng = np.random.default_rng(0)
    q, kc, vc, tables, lengths = random_case(rng, [0, 1, 3, 4, 5, 17, 40])
    actual = ref.paged_attention(q, kc, vc, tables, lengths)
    expected = sdpa_rows(q, history(kc, tables, lengths), history(vc, tables, lengths), 2)
    np.testing.assert_allclose(actual, expected, atol=2e-6, rtol=2e-5)


def test_window_equals_sliced_history():
    rng = np.random.default_rng(1)
    q, kc, vc, tables, lengths = random_case(rng, [0, 1, 6, 9, 30])
    for window in (1, 2, 7, 100):
        start = [max(0, n - window) for n in lengths]
        actual = ref.paged_attention(q, kc, vc, tables, lengths, window=window)
        expected = sdpa_rows(q, history(kc, tables, lengths, start),
                             history(vc, tables, lengths, start), 2)
        np.testing.assert_allclose(actual, expected, atol=2e-6, rtol=2e-5)


def test_closed_forms():
    rng = np.random.default_rng(2)
    q, kc, vc, tables, _ = random_case(rng, [8, 8])
    lengths = np.array([1, 0], np.int32)
    out = ref.paged_attention(q, kc, vc, tables, lengths)
    np.testing.assert_array_equal(out[0], np.repeat(vc[tables[0, 0], 0], 2, axis=0))
    assert not out[1].any()
    kc[:] = 0.75  # constant keys: uniform weights
    lengths = np.array([7, 8], np.int32)
    out = ref.paged_attention(q, kc, vc, tables, lengths)
    for row in range(2):
        mean = history(vc, tables, lengths)[row].mean(axis=0)
        np.testing.assert_allclose(out[row], np.repeat(mean, 2, axis=0), atol=1e-6)


def test_early_exit_closed_form_means():
    """tests/test_kv_cache.py:61-77 restated: value at (p, d, layer) is
    100 + 10p + min(p, d) + layer with zero queries -> plain mean."""
    layer, block = 1, 2
    for position, depth in [(0, 0), (1, 1), (2, 2), (2, 1)]:
        n = position + 1
        vc = np.zeros((2, block, 1, 4), np.float32)
        for p in range(n):
            vc[p // block, p % block] = 100 + 10 * p + min(p, depth) + layer
        kc = np.ones_like(vc)
        tables = np.array([[0, 1]], np.int32)
        out = ref.paged_attention(np.zeros((1, 2, 4), np.float32), kc, vc, tables,
                                  np.array([n], np.int32))
        expected = np.mean([100 + 10 * p + min(p, depth) + layer for p in range(n)])
        np.testing.assert_allclose(out, np.full_like(out, expected), rtol=1e-6)


def test_prefill_rows_are_bottom_right_aligned():
    tables, lengths = ref.prefill_rows(np.array([[1, 2], [3, 4]], np.int32),
                                       np.array([5, 3], np.int32), np.array([0, 2, 5]))
    assert lengths.tolist() == [4, 5, 1, 2, 3]
    assert tables[:, 0].tolist() == [1, 1, 3, 3, 3]


def test_prefill_matches_causal_sdpa():
    rng = np.random.default_rng(3)
    dim, block, heads = 8, 4, 2
    n, q_len = 11, 5
    kc = rng.standard_normal((4, block, heads, dim)).astype(np.float32)
    vc = rng.standard_normal((4, block, heads, dim)).astype(np.float32)
    tables = np.array([[2, 0, 3]], np.int32)
    q = rng.standard_normal((q_len, heads, dim)).astype(np.float32)
    out = ref.paged_prefill(q, kc, vc, tables, np.array([n], np.int32), np.array([0, q_len]))
    keys = torch.from_numpy(history(kc, tables, [n])[0]).transpose(0, 1)
    values = torch.from_numpy(history(vc, tables, [n])[0]).transpose(0, 1)
    mask = torch.arange(n)[None, :] <= (n - q_len + torch.arange(q_len))[:, None]
    expected = F.scaled_dot_product_attention(torch.from_numpy(q).transpose(0, 1), keys, values,
                                              attn_mask=mask)
    np.testing.assert_allclose(out, expected.transpose(0, 1).numpy(), atol=2e-6, rtol=2e-5)


@pytest.mark.parametrize("groups", [1, 4])
def test_causal_block_matches_row_oracle_and_sdpa(groups):
    """causal_block (whole query tiles at once) equals paged_attention on the
    per-query rows, and SDPA with the causal mask; a wrong mask offset, head
    mapping or scale fails one of them."""
    rng = np.random.default_rng(21 + groups)
    dim, block, kv_heads = 16, 4, 2
    heads = kv_heads * groups
    n, q_len = 37, 9
    pages = -(-n // block)
    kc = rng.standard_normal((pages + 3, block, kv_heads, dim)).astype(np.float32)
    vc = rng.standard_normal((pages + 3, block, kv_heads, dim)).astype(np.float32)
    table = rng.permutation(pages + 3)[:pages].astype(np.int32)
    q = rng.standard_normal((q_len, heads, dim)).astype(np.float32)
    keys = history(kc, table[None], [n])[0]
    values = history(vc, table[None], [n])[0]
    positions = n - q_len + np.arange(q_len)
    got = ref.causal_block(q, keys, values, positions)
    rows = ref.paged_prefill(q, kc, vc, table[None], np.array([n], np.int32),
                             np.array([0, q_len]))
    np.testing.assert_allclose(got, rows, atol=1e-6, rtol=1e-5)
    kt = torch.from_numpy(np.repeat(keys, groups, axis=1)).transpose(0, 1)
    vt = torch.from_numpy(np.repeat(values, groups, axis=1)).transpose(0, 1)
    mask = torch.arange(n)[None, :] <= torch.from_numpy(positions)[:, None]
    expected = F.scaled_dot_product_attention(torch.from_numpy(q).transpose(0, 1), kt, vt,
                                              attn_mask=mask)
    np.testing.assert_allclose(got, expected.transpose(0, 1).numpy(), atol=2e-6, rtol=2e-5)
    # a query at position 0 sees one key: its output is that value row
    first = ref.causal_block(q[:1], keys, values, [0])
    np.testing.assert_allclose(first[0], np.repeat(values[0], groups, axis=0), atol=1e-6)


def test_bf16_rounding_matches_torch():
    x = np.random.default_rng(4).standard_normal(10000).astype(np.float32) * 100
    x[:4] = [np.inf, -np.inf, 0.0, -0.0]
    ours = ref.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)
    assert np.array_equal(ours, theirs)
    np.testing.assert_array_equal(ref.bf16_bits_to_f32(ours),
                                  torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_golden_fixture_reproduces():
    data = np.load(os.path.join(GOLDEN, "decode_small.npz"))
    out = ref.paged_attention(data["q"], data["k"], data["v"], data["tables"], data["lengths"])
    np.testing.assert_allclose(out, data["out"], atol=1e-6, rtol=1e-6)
    groups = data["q"].shape[1] // data["k"].shape[2]
    expected = sdpa_rows(data["q"], history(data["k"], data["tables"], data["lengths"]),
                         history(data["v"], data["tables"], data["lengths"]), groups)
    np.testing.assert_allclose(data["out"], expected, atol=2e-6, rtol=2e-5)


def test_integer_kernels_brute_force():
    rng = np.random.default_rng(5)
    tables = rng.integers(0, 1000, (5, 6)).astype(np.int32)
    positions = rng.integers(0, 96, 40)
    sequences = rng.integers(0, 5, 40)
    blocks, offsets = ref.expand_kv_addresses(positions, sequences, tables, 16)
    for i in range(40):
        assert blocks[i] == tables[sequences[i]][positions[i] // 16]
        assert offsets[i] == positions[i] - 16 * (positions[i] // 16)
    # metadata_kernel literal case: slot 1, depth 2, pos 17 of a 3-plane table.
    route = np.arange(2 * 3 * 4, dtype=np.int32).reshape(6, 4) + 100
    out = ref.routing_metadata(np.array([[1, 2, 17]]), route, n=1, size=2, width=4, page=16,
                               planes=3, out_width=3)
    assert out["blocks"].tolist()[0] == 100 + (1 * 3 + 2) * 4 + 1
    assert out["lengths"].tolist() == [18, 0]
    assert out["out_tables"].tolist() == [[120, 121, 122, -1], [0, 0, 0, -1]]
    assert ref.routing_slots(np.array([[7, 0, 0], [3, 1, 1]]), 2, 3).tolist() == [7, 3, 0]


def test_kv_movement_closed_forms():
    pool_k = np.arange(4 * 2 * 2 * 1 * 3, dtype=np.float32).reshape(4, 2, 2, 1, 3)
    pool_v = -pool_k
    tables = np.array([[0, 1], [2, 3]], np.int32)  # slot 0: plane 0 = [0, 1], plane 1 = [2, 3]
    k2, v2 = pool_k.copy(), pool_v.copy()
    ref.finalize_rows(k2, v2, np.array([[0, 0, 3]]), tables, planes=2)
    np.testing.assert_array_equal(k2[3, :, 1], pool_k[1, :, 1])
    changed = (k2 != pool_k)
    assert changed[3, :, 1].all() and changed.sum() == changed[3, :, 1].size
    k3, v3 = pool_k.copy(), pool_v.copy()
    ref.copy_blocks(k3, v3, [0], [2])
    np.testing.assert_array_equal(k3[2], pool_k[0])
    np.testing.assert_array_equal(v3[2], pool_v[0])
    keys, values = ref.kv_gather(pool_k[:, 1], pool_v[:, 1], [3, 0], 3)
    np.testing.assert_array_equal(keys, np.stack([pool_k[3, 1, 0], pool_k[3, 1, 1],
                                                  pool_k[0, 1, 0]]))
    kc = np.zeros((3, 2, 1, 2), np.float32)
    vc = np.zeros_like(kc)
    k = np.arange(6, dtype=np.float32).reshape(3, 1, 2)
    ref.kv_append(kc, vc, k, -k, [2, 0, 1], [1, 0, 1], write_mask=[1, 1, 0], active_rows=2)
    np.testing.assert_array_equal(kc[2, 1], k[0])
    np.testing.assert_array_equal(kc[0, 0], k[1])
    assert not kc[1].any()
    assert math.isclose(float(vc[2, 1, 0, 1]), -1.0)


@pytest.mark.parametrize("seed", [0, 1])
def test_oracle_handles_fp16_widening(seed):
    rng = np.random.default_rng(seed)
    q, kc, vc, tables, lengths = random_case(rng, [5, 9])
    half = [x.astype(np.float16).astype(np.float32) for x in (q, kc, vc)]
    out = ref.paged_attention(*half, tables, lengths)
    assert out.dtype == np.float32 and np.isfinite(out).all()


# ------------------------------------------------------------ SiLU-and-Mul
def test_silu_oracle_known_values():
    # tests/test_activation.py:49-53 of the reference
    from oracle import activation_ref as act

    out = act.silu_and_mul(np.array([0.0, 1.0, -1.0], np.float32),
                           np.array([2.0, 3.0, 4.0], np.float32), "f32")
    np.testing.assert_allclose(out, [0.0, 2.1931758, -1.0757657], rtol=1e-6)


def test_silu_oracle_matches_torch_float64_and_odd_identity():
    from oracle import activation_ref as act

    x = np.concatenate([np.linspace(-120, 120, 4001), [0.0, -0.0, 1e-30, -1e-30, 745.0, -745.0]])
    ref64 = torch.nn.functional.silu(torch.tensor(x, dtype=torch.float64)).numpy()
    got = act.silu_f64(x)
    np.testing.assert_allclose(got, ref64, rtol=1e-14, atol=1e-300)  # x = -745: subnormal vs 0
    # silu(x) - silu(-x) = x * (sigmoid(x) + sigmoid(-x)) = x: a sign or branch slip breaks it
    np.testing.assert_allclose(got - act.silu_f64(-x), x, rtol=1e-12, atol=1e-300)
    special = act.silu_f64(np.array([np.inf, -np.inf, np.nan]))
    assert special[0] == np.inf and np.isnan(special[1]) and np.isnan(special[2])


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_silu_oracle_rounding_matches_torch_conversion_on_every_pattern(dtype):
    # torch rounds float64 -> storage dtype through float32; the oracle must too,
    # and the product path rounds once more (tests/test_activation.py:60-64).
    from oracle import activation_ref as act

    tdtype = torch.bfloat16 if dtype == "bf16" else torch.float16
    patterns = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(tdtype)
    gate = patterns.float().numpy()
    up = np.full_like(gate, 1.5, dtype=np.float32)
    g64 = patterns.double()
    expected_act = (g64 * torch.sigmoid(g64)).to(tdtype)
    expected = (expected_act.double() * 1.5).to(tdtype).float().numpy()
    got = act.silu_and_mul(gate, up, dtype)
    finite = ~np.isnan(expected)
    assert np.array_equal(np.isnan(got), ~finite)
    assert np.array_equal(got[finite].view(np.uint32), expected[finite].view(np.uint32))


# ------------------------------------------------------- hidden-state rows
def test_row_and_segment_oracle_literal_vectors():
    pool = np.arange(24, dtype=np.int64).reshape(8, 3)
    out = ref.gather_rows(pool, np.array([5, 0, 7, 9]), 3, 4)
    assert out.tolist() == [[15, 16, 17], [0, 1, 2], [21, 22, 23], [0, 0, 0]]
    target = np.zeros((8, 3), np.int64)
    ref.scatter_rows(np.array([[1, 2, 3], [4, 5, 6]]), np.array([6, 1]), target, 2)
    assert target[6].tolist() == [1, 2, 3] and target[1].tolist() == [4, 5, 6]
    assert target.sum() == 21
    # two state slots of 4 rows each; segments (slot, offset, count, start, keep)
    segments = np.array([[1, 1, 2, 0, 1], [0, 3, 1, 2, 0]])
    batch = np.full((3, 3), -1, np.int64)
    ref.gather_segments(pool, segments, batch, 4)
    assert batch.tolist() == [[15, 16, 17], [18, 19, 20], [9, 10, 11]]
    back = np.zeros_like(pool)
    ref.scatter_segments(batch, segments, back, 4)
    assert back[5].tolist() == [15, 16, 17] and back[6].tolist() == [18, 19, 20]
    assert back[3].tolist() == [0, 0, 0]  # keep = 0: not stored


def test_torch_cpu_restatement_matches_numpy_oracle():
    # the CPU baseline's Torch restatement must compute the oracle's function
    from oracle import torch_ref

    gen = torch.Generator().manual_seed(4)
    kc = torch.randn(12, 4, 2, 8, generator=gen)
    vc = torch.randn(12, 4, 2, 8, generator=gen)
    q = torch.randn(3, 4, 8, generator=gen)
    tables = torch.tensor([[5, 1, 9], [0, 0, 0], [11, 3, 7]], dtype=torch.int32)
    lengths = torch.tensor([10, 0, 12], dtype=torch.int32)
    got = torch_ref.paged_attention(q, kc, vc, tables, lengths)
    want = ref.paged_attention(q.numpy(), kc.numpy(), vc.numpy(), tables.numpy(), lengths.numpy())
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-6)
    # packed prefill as decode rows, against the numpy oracle's own expansion
    cu = torch.tensor([0, 4, 5, 7], dtype=torch.int32)
    qp = torch.randn(7, 4, 8, generator=gen)
    got = torch_ref.prefill(qp, kc, vc, tables, lengths, cu)
    want = ref.paged_prefill(qp.numpy(), kc.numpy(), vc.numpy(), tables.numpy(),
                             lengths.numpy(), cu.numpy())
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-5, atol=1e-6)
    # the index-put append is the oracle's append on the layer view (bit-exact)
    pool_k = torch.randn(6, 3, 4, 2, 8, generator=gen)
    pool_v = torch.randn(6, 3, 4, 2, 8, generator=gen)
    k_new = torch.randn(5, 2, 8, generator=gen)
    blocks = torch.tensor([4, 0, 4, 2, 5])
    offsets = torch.tensor([1, 3, 2, 0, 3])
    want_k, want_v = pool_k[:, 1].numpy().copy(), pool_v[:, 1].numpy().copy()
    ref.kv_append(want_k, want_v, k_new.numpy(), -k_new.numpy(), blocks.numpy(), offsets.numpy())
    torch_ref.append(pool_k, pool_v, 1, k_new, -k_new, blocks, offsets)
    assert np.array_equal(pool_k[:, 1].numpy(), want_k)
    assert np.array_equal(pool_v[:, 1].numpy(), want_v)


def test_expand_kv_addresses_literal_packed_vectors():
    """tests/test_flash_attention.py:121-143: two packed sequences with
    positions [7, 8, 9] and [3, 4] on 4-token pages (context lengths [10, 5],
    cu_seqlens_q [0, 3, 5]); blocks and offsets written out by hand for the
    tables [10, 11, 12] and [20, 21]."""
    tables = np.array([[10, 11, 12], [20, 21, -1]], np.int32)
    blocks, offsets = ref.expand_kv_addresses([7, 8, 9, 3, 4], [0, 0, 0, 1, 1], tables, 4)
    assert blocks.tolist() == [11, 12, 12, 20, 21]
    assert offsets.tolist() == [3, 0, 1, 3, 0]
    rows, lengths = ref.prefill_rows(tables, np.array([10, 5]), np.array([0, 3, 5]))
    assert lengths.tolist() == [8, 9, 10, 4, 5]  # position + 1 of each packed query
    # a page size of 1 makes every position its own page
    blocks, offsets = ref.expand_kv_addresses([2, 0], [1, 0], tables, 1)
    assert blocks.tolist() == [-1, 10] and offsets.tolist() == [0, 0]


def test_finalize_token_closed_form():
    """tests/test_kv_cache.py:38-58: token 0 of a 3-plane request is written at
    depths 0 and 1 of both layers with keys 10 * layer + depth (values + 100)
    and exits at depth 1. Plane 2 then holds depth 1's keys and values in
    every layer, plane 0 keeps its own, and nothing else changes."""
    blocks, layers, bs = 6, 2, 2
    key_pool = np.full((blocks, layers, bs, 1, 4), -7.0, np.float32)
    value_pool = key_pool.copy()
    plane_block = {0: 4, 1: 1, 2: 3}  # page 0 of each plane
    for layer in range(layers):
        for depth in (0, 1):
            key_pool[plane_block[depth], layer, 0] = 10 * layer + depth
            value_pool[plane_block[depth], layer, 0] = 10 * layer + depth + 100
    k0, v0 = key_pool.copy(), value_pool.copy()
    ref.finalize_token(key_pool, value_pool, plane_block[1], [plane_block[2]], 0, [0, 1])
    for layer in range(layers):
        np.testing.assert_array_equal(key_pool[3, layer, 0], np.full((1, 4), 10 * layer + 1.0))
        np.testing.assert_array_equal(value_pool[3, layer, 0], np.full((1, 4), 10 * layer + 101.0))
        np.testing.assert_array_equal(key_pool[4, layer, 0], np.full((1, 4), 10.0 * layer))
    changed = key_pool != k0
    assert changed.sum() == changed[3, :, 0].size and changed[3, :, 0].all()
    assert ((value_pool != v0).sum()) == changed.sum()
    # physical copies: a later write at depth 1 does not reach plane 2
    key_pool[1, 0, 0] = 0.0
    np.testing.assert_array_equal(key_pool[3, 0, 0], np.ones((1, 4)))
    # an empty layer list or destination list changes nothing
    k1 = key_pool.copy()
    ref.finalize_token(key_pool, value_pool, 1, [], 0, [0, 1])
    ref.finalize_token(key_pool, value_pool, 1, [5], 0, [])
    np.testing.assert_array_equal(key_pool, k1)


def test_snapshot_round_trip_and_page_count_refusal():
    """tests/test_kv_cache.py:261-303: pages go to host rows in table order and
    come back into other blocks of a disturbed pool, byte for byte; a
    snapshot is refused by a restore target with another page count."""
    shape = (8, 2, 2, 1, 3)
    slot = int(np.prod(shape[1:]))
    key_pool = np.arange(np.prod(shape), dtype=np.float32).reshape(shape)
    value_pool = -key_pool - 1
    keys, values = ref.blocks_to_host(key_pool, value_pool, [5, 2, 7])
    for row, block in enumerate([5, 2, 7]):
        np.testing.assert_array_equal(keys[row].ravel(), block * slot + np.arange(slot))
        np.testing.assert_array_equal(values[row].ravel(), -(block * slot + np.arange(slot)) - 1)
    keys_before = keys.copy()
    key_pool[5] = 0.0  # the host rows are copies, not views
    np.testing.assert_array_equal(keys, keys_before)
    target_k = np.full(shape, 9.0, np.float32)
    target_v = target_k.copy()
    ref.blocks_from_host(target_k, target_v, [1, 0, 3], keys, values)
    for row, block in enumerate([1, 0, 3]):
        np.testing.assert_array_equal(target_k[block], keys_before[row])
        np.testing.assert_array_equal(target_v[block], values[row])
    untouched = [b for b in range(8) if b not in (1, 0, 3)]
    assert (target_k[untouched] == 9.0).all() and (target_v[untouched] == 9.0).all()
    with pytest.raises(ValueError, match="page count"):
        ref.blocks_from_host(target_k, target_v, [1, 0], keys, values)
    with pytest.raises(ValueError, match="page count"):
        ref.blocks_from_host(target_k, target_v, [1, 0, 3, 4], keys, values)
