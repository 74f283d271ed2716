"""KV metadata contracts and their host construction.

Same contracts as the reference's vllm_rlt/worker/metadata.py:21-229:
  * ``KVMetadata``: host-validated rows plus device tensors for one traversal:
    positions / write_blocks / write_offsets int64 ``[rows]``, block_tables int32
    ``[rows or sequences, width]`` contiguous, context_lengths int32, optional
    cu_seqlens_q int32 ``[sequences + 1]``.
  * ``DeviceKVMetadata``: the stream-ordered variant whose positions are owned
    by the GPU (async routing); ``write_mask`` bool ``[rows]``, ``active_rows``
    an int32 device scalar for bucketed graph rows.
  * ``MetadataBuilder.build`` resolves (request, depth, position) rows to the
    depth plane's physical page, rejects aliased writes, and plans attention
    metadata; staging uploads one int64 and one int32 buffer
    (worker/buffers.py:153-199).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import TYPE_CHECKING

import torch

from vllm_rlt.attention.metadata import AttentionRows, plan_attention_metadata

if TYPE_CHECKING:
    from vllm_rlt.core.kv_cache_manager import KVCacheManager


@dataclass(frozen=True, eq=False)
class KVMetadata:
    owner: KVCacheManager
    rows: tuple
    allocations: tuple
    position_ids: torch.Tensor
    write_blocks: torch.Tensor
    write_offsets: torch.Tensor
    block_tables: torch.Tensor
    context_lengths: torch.Tensor
    writable: bool
    cu_seqlens_q: torch.Tensor | None = None
    max_seqlen_q: int = 1


@dataclass(frozen=True, eq=False)
class DeviceKVMetadata:
    allocations: tuple
    position_ids: torch.Tensor
    write_blocks: torch.Tensor
    write_offsets: torch.Tensor
    block_tables: torch.Tensor
    context_lengths: torch.Tensor
    write_mask: torch.Tensor | None = None
    active_rows: torch.Tensor | None = None
    cu_seqlens_q: torch.Tensor | None = None
    max_seqlen_q: int = 1


class MetadataBuilder:
    def __init__(self, cache: KVCacheManager):
        self.cache = cache

    def prepare_device(self, *, allocations, position_ids, write_blocks, write_offsets,
                       block_tables, context_lengths, write_mask=None,
                       active_rows=None) -> DeviceKVMetadata:
        """Borrow stream-ordered metadata without reading device values on the host."""
        cache = self.cache
        batch = DeviceKVMetadata(
            allocations=tuple(allocations),
            position_ids=position_ids,
            write_blocks=write_blocks,
            write_offsets=write_offsets,
            block_tables=block_tables,
            context_lengths=context_lengths,
            write_mask=write_mask,
            active_rows=active_rows,
        )
        if write_mask is not None and (
            write_mask.shape != position_ids.shape
            or write_mask.dtype != torch.bool
            or write_mask.device != cache.device
        ):
            raise ValueError("write_mask must be bool [rows] on the cache device")
        if active_rows is not None and (
            active_rows.dtype != torch.int32 or active_rows.numel() != 1
            or active_rows.device != cache.device
        ):
            raise ValueError("active_rows must be an int32 scalar on the cache device")
        cache._require_live_batch(batch)
        rows = len(position_ids)
        for name, tensor, dtype in (
            ("position_ids", position_ids, torch.int64),
            ("write_blocks", write_blocks, torch.int64),
            ("write_offsets", write_offsets, torch.int64),
            ("context_lengths", context_lengths, torch.int32),
        ):
            if tensor.shape != (rows,) or tensor.dtype != dtype or tensor.device != cache.device:
                raise ValueError(
                    f"{name} must have shape [rows] and use {dtype} on {cache.device}"
                )
        if (
            not allocations
            or block_tables.ndim != 2
            or block_tables.shape[0] != rows
            or block_tables.shape[1] == 0
            or block_tables.dtype != torch.int32
            or block_tables.device != cache.device
            or not block_tables.is_contiguous()
        ):
            raise ValueError("device block tables must be contiguous int32 [rows, pages]")
        return batch

    def write_addresses(self, rows, *, for_write=True):
        """Physical (page, offset) of each row; aliased writes are rejected."""
        cache = self.cache
        blocks = [
            allocation.block_tables[cache._plane(depth)][position // cache.block_size]
            for allocation, depth, position in rows
        ]
        offsets = [position % cache.block_size for _, _, position in rows]
        if for_write and len(set(zip(blocks, offsets))) != len(rows):
            raise ValueError("duplicate KV write addresses for request/depth/position rows")
        return blocks, offsets

    def build(self, request_ids, depths, positions, *, packed=False,
              for_write=True) -> KVMetadata:
        cache = self.cache
        if packed and (cache.layout != "last_exited"
                       or not cache.attention_capabilities.packed_prefill):
            raise ValueError("packed queries require a compatible attention backend and KV layout")
        rows = tuple(cache._validate_rows(request_ids, depths, positions))
        blocks, offsets = self.write_addresses(rows, for_write=for_write)
        positions = [p for _, _, p in rows]
        plan = plan_attention_metadata(
            AttentionRows(
                block_tables=[a.block_tables[cache._plane(d)] for a, d, _ in rows],
                positions=positions,
                sequence_keys=[(id(a), d) for a, d, _ in rows] if packed else None,
            ),
            block_size=cache.block_size,
            packed_prefill=packed,
        )
        n, t, width = len(rows), plan.num_rows, plan.table_width
        wide = cache._stage(positions + blocks + offsets, torch.int64)
        narrow = cache._stage(
            plan.block_tables + plan.context_lengths + (plan.cu_seqlens_q or []), torch.int32
        )
        allocations = tuple(dict(zip(request_ids, (a for a, _, _ in rows))).items())
        return KVMetadata(
            owner=cache,
            rows=rows,
            allocations=allocations,
            position_ids=wide[:n],
            write_blocks=wide[n : 2 * n],
            write_offsets=wide[2 * n : 3 * n],
            block_tables=narrow[: t * width].view(t, width),
            context_lengths=narrow[t * width : t * width + t],
            writable=for_write,
            cu_seqlens_q=(
                narrow[t * width + t : t * width + 2 * t + 1]
                if plan.cu_seqlens_q is not None
                else None
            ),
            max_seqlen_q=plan.max_seqlen_q,
        )
