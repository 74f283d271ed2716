"""Seeded synthetic workloads at the benchmark configurations' shapes.

Generators: ``torch.Generator`` seeded 0 for page placement (tables), 1 for
values, 2 for lengths/depths. Block tables are a seeded permutation of the
physical pool, so every row's pages are scattered. Padding entries are -1.

Configurations (shape symbols: Hq = Hkv = 16, D = 128, block_size 16):
  1  8 rows, context ~ U[64, 512], one new token appended at position n then
     attended with length n + 1; fp32; single-layer pool.
  2  Ouro-1.4B decode over a LAST_EXITED pool: 64 requests x 4 depth planes,
     24 layers, context ~ U[512, 4096], each row at depth ~ U{0..3}, bf16
     N(0,1) * 0.5; appends at position n of the row's plane, decode length n+1.
  3  SHARED layout with prefix reuse: 128 requests in 16 groups of 8 sharing a
     1024-token (64-page) prefix, private suffix ~ U[64, 1024]; appends land
     mid-page; bf16 N(0,1).
  4  WCPB prefill + decode: 16 prompts ~ U[1024, 8192] in 512-token chunks, one
     chunk per prompt at a random chunk index and depth ~ U{0..3}, prefix =
     index * 512 at that depth; plus 48 decode rows with context ~ U[256, 4096].
  5  Ouro-2.6B decode shape: 256 rows, context ~ U[2048, 32768], a 48-layer
     pool (6 MiB of K+V per block in bf16) of ``pool_blocks`` blocks and
     2048-page tables. The resident context (~4.4M tokens x 48 layers) exceeds
     any one GPU, so rows draw their pages from the pool at random: each row's
     pages are distinct, rows may share pages (the per-row bytes are counted
     as read, as for shared prefixes). Appends land at position n - 1 of each
     row (its last page).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

HEADS = 16
HEAD_DIM = 128
BLOCK = 16


def _gens():
    return tuple(torch.Generator().manual_seed(s) for s in (0, 1, 2))


def _randint(gen, low, high, size):
    return torch.randint(low, high + 1, (size,), generator=gen)


@dataclass
class DecodeWorkload:
    """One decode step: append rows' K/V, then attend with length n + 1."""

    name: str
    dtype: torch.dtype
    layers: int
    num_blocks: int
    key_cache: torch.Tensor          # [N, L, bs, H, D]
    value_cache: torch.Tensor
    q: torch.Tensor                  # [rows, Hq, D]
    k_new: torch.Tensor              # [L, rows, H, D] appended K (per layer)
    v_new: torch.Tensor
    block_tables: torch.Tensor       # int32 [rows, W] (-1 padded), the row's plane
    context_lengths: torch.Tensor    # int32 [rows] (after the append)
    write_blocks: torch.Tensor       # int64 [rows]
    write_offsets: torch.Tensor      # int64 [rows]
    extra: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return self.q.shape[0]

    def decode_bytes(self) -> int:
        """Algorithmic bytes of one per-layer decode call: K+V of every visible
        token per row, q in and out, and the page-table entries read."""
        es = self.key_cache.element_size()
        hkv, d = self.key_cache.shape[3], self.key_cache.shape[4]
        lengths = self.context_lengths.to(torch.int64)
        kv = int(lengths.sum()) * 2 * hkv * d * es
        qo = 2 * self.q.numel() * es
        tables = int(((lengths + BLOCK - 1) // BLOCK).sum()) * 4
        return kv + qo + tables

    def append_bytes(self, layers: int = 1) -> int:
        """Algorithmic bytes of appending ``layers`` layers: K+V read and written,
        plus 16 B of addresses per row."""
        es = self.key_cache.element_size()
        slot = self.k_new.shape[2] * self.k_new.shape[3] * es
        return layers * self.rows * 2 * slot * 2 + self.rows * 16


def _scatter_pages(gen_tables, counts, num_blocks):
    """Assign each entry of ``counts`` its pages from one seeded permutation."""
    order = torch.randperm(num_blocks, generator=gen_tables).tolist()
    tables, cursor = [], 0
    for count in counts:
        tables.append(order[cursor : cursor + count])
        cursor += count
    return tables


def _table_tensor(tables, width):
    out = torch.full((len(tables), width), -1, dtype=torch.int32)
    for row, pages in enumerate(tables):
        out[row, : len(pages)] = torch.tensor(pages, dtype=torch.int32)
    return out


def _values(gen, shape, dtype, scale, device):
    x = torch.randn(shape, generator=gen, dtype=torch.float32)
    if scale != 1.0:
        x = x * scale
    return x.to(dtype).to(device)


def _fill_pool(pool, gen, scale, chunk_blocks=256):
    """Fill a pool with seeded N(0,1)*scale values, chunk by chunk on the device
    (a CPU generator seeds a device generator so large pools stay fast)."""
    seed = int(torch.randint(0, 2**62, (1,), generator=gen))
    device_gen = torch.Generator(device=pool.device).manual_seed(seed)
    for start in range(0, pool.shape[0], chunk_blocks):
        part = pool[start : start + chunk_blocks]
        part.normal_(0.0, scale, generator=device_gen)


def config1(device="cpu", rows=8, dtype=torch.float32) -> DecodeWorkload:
    g_tab, g_val, g_len = _gens()
    ctx = _randint(g_len, 64, 512, rows)
    lengths = ctx + 1
    pages = ((lengths + BLOCK - 1) // BLOCK).tolist()
    num_blocks = sum(pages)
    tables = _scatter_pages(g_tab, pages, num_blocks)
    width = max(pages)
    shape = (num_blocks, 1, BLOCK, HEADS, HEAD_DIM)
    key_cache = _values(g_val, shape, dtype, 1.0, device)
    value_cache = _values(g_val, shape, dtype, 1.0, device)
    q = _values(g_val, (rows, HEADS, HEAD_DIM), dtype, 1.0, device)
    k_new = _values(g_val, (1, rows, HEADS, HEAD_DIM), dtype, 1.0, device)
    v_new = _values(g_val, (1, rows, HEADS, HEAD_DIM), dtype, 1.0, device)
    wb = torch.tensor([tables[r][int(ctx[r]) // BLOCK] for r in range(rows)], dtype=torch.int64)
    wo = ctx.to(torch.int64) % BLOCK
    return DecodeWorkload("config1", dtype, 1, num_blocks, key_cache, value_cache, q, k_new,
                          v_new, _table_tensor(tables, width).to(device),
                          lengths.to(torch.int32).to(device), wb.to(device), wo.to(device))


def config2(device="cpu", rows=64, layers=24, depths=4, ctx_low=512, ctx_high=4096,
            dtype=torch.bfloat16, fill=True) -> DecodeWorkload:
    """LAST_EXITED: every request owns ``depths`` planes of ceil((n+1)/16) pages."""
    g_tab, g_val, g_len = _gens()
    ctx = _randint(g_len, ctx_low, ctx_high, rows)
    depth = _randint(g_len, 0, depths - 1, rows)
    lengths = ctx + 1
    pages = ((lengths + BLOCK - 1) // BLOCK).tolist()
    counts = [p for p in pages for _ in range(depths)]
    num_blocks = sum(counts)
    plane_tables = _scatter_pages(g_tab, counts, num_blocks)
    tables = [plane_tables[r * depths + int(depth[r])] for r in range(rows)]
    width = max(pages)
    shape = (num_blocks, layers, BLOCK, HEADS, HEAD_DIM)
    key_cache = torch.empty(shape, dtype=dtype, device=device)
    value_cache = torch.empty_like(key_cache)
    if fill:
        _fill_pool(key_cache, g_val, 0.5)
        _fill_pool(value_cache, g_val, 0.5)
    q = _values(g_val, (rows, HEADS, HEAD_DIM), dtype, 0.5, device)
    k_new = _values(g_val, (layers, rows, HEADS, HEAD_DIM), dtype, 0.5, device)
    v_new = _values(g_val, (layers, rows, HEADS, HEAD_DIM), dtype, 0.5, device)
    wb = torch.tensor([tables[r][int(ctx[r]) // BLOCK] for r in range(rows)], dtype=torch.int64)
    wo = ctx.to(torch.int64) % BLOCK
    return DecodeWorkload("config2", dtype, layers, num_blocks, key_cache, value_cache, q, k_new,
                          v_new, _table_tensor(tables, width).to(device),
                          lengths.to(torch.int32).to(device), wb.to(device), wo.to(device),
                          extra={"depths": depth, "plane_tables": plane_tables})


def config3(device="cpu", groups=16, per_group=8, prefix_pages=64, suffix_low=64,
            suffix_high=1024, layers=1, dtype=torch.bfloat16, fill=True,
            spare_blocks=0) -> DecodeWorkload:
    """SHARED layout: each group's requests alias the same prefix pages.
    ``spare_blocks`` free blocks follow the assigned ones (copy-on-write targets)."""
    g_tab, g_val, g_len = _gens()
    rows = groups * per_group
    suffix = _randint(g_len, suffix_low, suffix_high, rows)
    ctx = prefix_pages * BLOCK + suffix
    lengths = ctx + 1
    private = [int((lengths[r] + BLOCK - 1) // BLOCK) - prefix_pages for r in range(rows)]
    counts = [prefix_pages] * groups + private
    num_blocks = sum(counts) + spare_blocks
    assigned = _scatter_pages(g_tab, counts + [spare_blocks], num_blocks)
    spare = assigned.pop()
    tables = [assigned[r // per_group] + assigned[groups + r] for r in range(rows)]
    width = max(len(t) for t in tables)
    shape = (num_blocks, layers, BLOCK, HEADS, HEAD_DIM)
    key_cache = torch.empty(shape, dtype=dtype, device=device)
    value_cache = torch.empty_like(key_cache)
    if fill:
        _fill_pool(key_cache, g_val, 1.0)
        _fill_pool(value_cache, g_val, 1.0)
    q = _values(g_val, (rows, HEADS, HEAD_DIM), dtype, 1.0, device)
    k_new = _values(g_val, (layers, rows, HEADS, HEAD_DIM), dtype, 1.0, device)
    v_new = _values(g_val, (layers, rows, HEADS, HEAD_DIM), dtype, 1.0, device)
    wb = torch.tensor([tables[r][int(ctx[r]) // BLOCK] for r in range(rows)], dtype=torch.int64)
    wo = ctx.to(torch.int64) % BLOCK
    unique_tokens = groups * prefix_pages * BLOCK + int(suffix.sum()) + rows
    return DecodeWorkload("config3", dtype, layers, num_blocks, key_cache, value_cache, q, k_new,
                          v_new, _table_tensor(tables, width).to(device),
                          lengths.to(torch.int32).to(device), wb.to(device), wo.to(device),
                          extra={"prefix_tables": assigned[:groups],
                                 "unique_tokens": unique_tokens, "spare_blocks": spare})


def config5(device="cpu", rows=256, ctx_low=2048, ctx_high=32768, layers=48,
            pool_blocks=32768, width=2048, dtype=torch.bfloat16, fill=True) -> DecodeWorkload:
    """Long-context decode over a 48-layer pool (see the module docstring)."""
    g_tab, g_val, g_len = _gens()
    lengths = _randint(g_len, ctx_low, ctx_high, rows)
    pages = ((lengths + BLOCK - 1) // BLOCK).tolist()
    if max(pages) > min(width, pool_blocks):
        raise ValueError("contexts exceed the table width or the pool")
    order = torch.randperm(pool_blocks, generator=g_tab)
    starts = torch.randint(0, pool_blocks, (rows,), generator=g_tab)
    tables = torch.full((rows, width), -1, dtype=torch.int32)
    for r in range(rows):
        idx = (int(starts[r]) + torch.arange(pages[r])) % pool_blocks
        tables[r, : pages[r]] = order[idx].to(torch.int32)
    shape = (pool_blocks, layers, BLOCK, HEADS, HEAD_DIM)
    key_cache = torch.empty(shape, dtype=dtype, device=device)
    value_cache = torch.empty_like(key_cache)
    if fill:
        _fill_pool(key_cache, g_val, 0.5)
        _fill_pool(value_cache, g_val, 0.5)
    q = _values(g_val, (rows, HEADS, HEAD_DIM), dtype, 0.5, device)
    k_new = _values(g_val, (1, rows, HEADS, HEAD_DIM), dtype, 0.5, device)
    v_new = _values(g_val, (1, rows, HEADS, HEAD_DIM), dtype, 0.5, device)
    last = (lengths - 1).to(torch.int64)
    wb = tables[torch.arange(rows), last // BLOCK].to(torch.int64)
    wo = last % BLOCK
    return DecodeWorkload("config5", dtype, layers, pool_blocks, key_cache, value_cache, q, k_new,
                          v_new, tables.to(device), lengths.to(torch.int32).to(device),
                          wb.to(device), wo.to(device))


def gqa_decode(device="cpu", rows=64, q_heads=32, kv_heads=8, ctx_low=512, ctx_high=4096,
               dtype=torch.bfloat16) -> DecodeWorkload:
    """Grouped-query decode (q_heads / kv_heads q heads per kv head) at config 2's
    row count and context range, over a one-layer pool of the rows' pages."""
    g_tab, g_val, g_len = _gens()
    lengths = _randint(g_len, ctx_low, ctx_high, rows) + 1
    pages = ((lengths + BLOCK - 1) // BLOCK).tolist()
    num_blocks = sum(pages)
    tables = _scatter_pages(g_tab, pages, num_blocks)
    shape = (num_blocks, 1, BLOCK, kv_heads, HEAD_DIM)
    key_cache = torch.empty(shape, dtype=dtype, device=device)
    value_cache = torch.empty_like(key_cache)
    _fill_pool(key_cache, g_val, 0.5)
    _fill_pool(value_cache, g_val, 0.5)
    q = _values(g_val, (rows, q_heads, HEAD_DIM), dtype, 0.5, device)
    empty = torch.empty((1, 0, kv_heads, HEAD_DIM), dtype=dtype, device=device)
    none = torch.empty(0, dtype=torch.int64, device=device)
    return DecodeWorkload("gqa", dtype, 1, num_blocks, key_cache, value_cache, q, empty, empty,
                          _table_tensor(tables, max(pages)).to(device),
                          lengths.to(torch.int32).to(device), none, none)


@dataclass
class PrefillWorkload:
    """Packed WCPB chunks + decode rows of config 4 (one layer)."""

    key_cache: torch.Tensor          # [N, 1, bs, H, D]
    value_cache: torch.Tensor
    q: torch.Tensor                  # [T, Hq, D]
    k_new: torch.Tensor              # [T, H, D] appended rows (chunks + decode)
    v_new: torch.Tensor
    block_tables: torch.Tensor       # int32 [S, W] per sequence
    context_lengths: torch.Tensor    # int32 [S]
    cu_seqlens_q: torch.Tensor       # int32 [S + 1]
    max_seqlen_q: int
    write_blocks: torch.Tensor       # int64 [T]
    write_offsets: torch.Tensor
    chunk_sequences: int

    def flops(self) -> int:
        """4 * D * Hq * sum over queries of visible keys."""
        cu = self.cu_seqlens_q.tolist()
        n = self.context_lengths.tolist()
        total = 0
        for s in range(len(n)):
            q_len = cu[s + 1] - cu[s]
            total += sum(n[s] - q_len + i + 1 for i in range(q_len))
        return 4 * self.q.shape[2] * self.q.shape[1] * total

    def append_bytes(self) -> int:
        rows = self.k_new.shape[0]
        slot = self.k_new.shape[1] * self.k_new.shape[2] * self.k_new.element_size()
        return rows * slot * 4 + rows * 16


def config4(device="cpu", prompts=16, decode_rows=48, chunk=512, dtype=torch.bfloat16,
            prompt_low=1024, prompt_high=8192, decode_low=256, decode_high=4096,
            fill=True) -> PrefillWorkload:
    g_tab, g_val, g_len = _gens()
    prompt_len = _randint(g_len, prompt_low, prompt_high, prompts)
    seqs = []  # (prefix, q_len)
    for p in range(prompts):
        chunks = -(-int(prompt_len[p]) // chunk)
        index = int(torch.randint(0, chunks, (1,), generator=g_len))
        _ = int(torch.randint(0, 4, (1,), generator=g_len))  # depth: selects the plane
        start = index * chunk
        seqs.append((start, min(chunk, int(prompt_len[p]) - start)))
    dec = _randint(g_len, decode_low, decode_high, decode_rows)
    for r in range(decode_rows):
        seqs.append((int(dec[r]), 1))
    lengths = [prefix + q for prefix, q in seqs]
    pages = [-(-n // BLOCK) for n in lengths]
    num_blocks = sum(pages)
    tables = _scatter_pages(g_tab, pages, num_blocks)
    width = max(pages)
    shape = (num_blocks, 1, BLOCK, HEADS, HEAD_DIM)
    key_cache = torch.empty(shape, dtype=dtype, device=device)
    value_cache = torch.empty_like(key_cache)
    if fill:
        _fill_pool(key_cache, g_val, 1.0)
        _fill_pool(value_cache, g_val, 1.0)
    total = sum(q for _, q in seqs)
    q = _values(g_val, (total, HEADS, HEAD_DIM), dtype, 1.0, device)
    k_new = _values(g_val, (total, HEADS, HEAD_DIM), dtype, 1.0, device)
    v_new = _values(g_val, (total, HEADS, HEAD_DIM), dtype, 1.0, device)
    cu = [0]
    wb, wo = [], []
    for s, (prefix, q_len) in enumerate(seqs):
        cu.append(cu[-1] + q_len)
        for i in range(q_len):
            pos = prefix + i
            wb.append(tables[s][pos // BLOCK])
            wo.append(pos % BLOCK)
    return PrefillWorkload(
        key_cache, value_cache, q, k_new, v_new, _table_tensor(tables, width).to(device),
        torch.tensor(lengths, dtype=torch.int32, device=device),
        torch.tensor(cu, dtype=torch.int32, device=device), max(q for _, q in seqs),
        torch.tensor(wb, dtype=torch.int64, device=device),
        torch.tensor(wo, dtype=torch.int64, device=device), prompts,
    )
