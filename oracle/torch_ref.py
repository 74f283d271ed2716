"""Torch-on-CPU restatement of the reference decode attention — TEST AND
BASELINE INFRASTRUCTURE ONLY.

Used by ``bench.py``'s ``cpu_baseline`` leg (timed with 1 and with k host
threads) and pinned against the numpy oracle in tests/test_oracle.py. The
product path never imports it.

Follows kernels/paged_attention.py:12-36 of the reference operation by
operation: per row, the visible tokens' keys/values are gathered through the
block table, KV heads are repeated for GQA, scores are fp32 dot products
scaled by 1/sqrt(D), softmax runs in fp32, the weighted sum of fp32 values is
rounded to the storage dtype; a length-0 row is zero.
"""

from __future__ import annotations

import math

import torch


def paged_attention(q, key_cache, value_cache, block_tables, context_lengths):
    rows, q_heads, dim = q.shape
    block = key_cache.shape[1]
    group = q_heads // key_cache.shape[2]
    scale = 1.0 / math.sqrt(dim)
    out = torch.empty_like(q)
    for row, n in enumerate(context_lengths.tolist()):
        if n == 0:
            out[row].zero_()
            continue
        pos = torch.arange(n)
        pages = block_tables[row].long()[pos // block]
        keys = key_cache[pages, pos % block]        # [n, kv_heads, D]
        values = value_cache[pages, pos % block]
        if group > 1:
            keys = keys.repeat_interleave(group, dim=1)
            values = values.repeat_interleave(group, dim=1)
        scores = torch.einsum("hd,nhd->hn", q[row].float(), keys.float()) * scale
        weights = torch.softmax(scores, dim=-1)
        out[row] = torch.einsum("hn,nhd->hd", weights, values.float()).to(q.dtype)
    return out


def append(key_cache, value_cache, layer, k, v, write_blocks, write_offsets):
    """The reference's eager append (core/kv_cache_manager.py:698-699): one
    advanced-index put per cache, ``cache[blocks, layer, offsets] = k``, on a
    whole pool ``[N, L, bs, H, D]``."""
    key_cache[write_blocks, layer, write_offsets] = k
    value_cache[write_blocks, layer, write_offsets] = v


def prefill(q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q):
    """Packed causal prefill as per-query decode rows (the expansion of the
    reference's tests/test_attention.py:333-346): query i of sequence s reads
    the sequence's table with length n_s - q_s + i + 1."""
    tables, lengths = [], []
    cu = cu_seqlens_q.tolist()
    for s, n in enumerate(context_lengths.tolist()):
        q_len = cu[s + 1] - cu[s]
        for i in range(q_len):
            tables.append(block_tables[s])
            lengths.append(max(0, n - q_len + i + 1))
    return paged_attention(q, key_cache, value_cache, torch.stack(tables),
                           torch.tensor(lengths, dtype=torch.int32))
