"""KV metadata tensors of one traversal, built from physical page lists.

The tensors and dtypes are the ones the reference's vllm_rlt/worker/metadata.py
hands to its kernels (:21-68, :119-150): positions / write_blocks /
write_offsets int64 ``[rows]``, block_tables int32 ``[rows or sequences,
width]`` contiguous, context_lengths int32, optional cu_seqlens_q int32
``[sequences + 1]``, and for the stream-ordered (device-owned) form a bool
``write_mask`` and an int32 ``active_rows`` device scalar. The reference
manager's own bookkeeping fields (owner, request rows, allocations: used for
its stale-batch checks) stay with that manager.

Each row arrives with the page list of its depth plane already selected (the
caller's LAST_EXITED or SHARED choice, reference kv_cache_manager.py:525-526).
The write address of a row is that list's page ``position // block_size`` at
offset ``position % block_size`` (reference worker/metadata.py:153-164); two
rows writing one slot are refused.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch

from vllm_rlt.attention.metadata import AttentionRows, plan_attention_metadata


@dataclass(frozen=True, eq=False)
class KVMetadata:
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
    position_ids: torch.Tensor
    write_blocks: torch.Tensor
    write_offsets: torch.Tensor
    block_tables: torch.Tensor
    context_lengths: torch.Tensor
    write_mask: torch.Tensor | None = None
    active_rows: torch.Tensor | None = None
    cu_seqlens_q: torch.Tensor | None = None
    max_seqlen_q: int = 1


def write_addresses(row_pages: Sequence[Sequence[int]], positions: Sequence[int],
                    block_size: int, *, for_write: bool = True):
    """(blocks, offsets) of each row; the row's pages must cover its position."""
    if len(row_pages) != len(positions):
        raise ValueError("row_pages and positions must have equal lengths")
    blocks, offsets = [], []
    for pages, position in zip(row_pages, positions):
        if position < 0 or position // block_size >= len(pages):
            raise ValueError(f"position {position} is outside the row's {len(pages)} pages")
        blocks.append(int(pages[position // block_size]))
        offsets.append(position % block_size)
    if for_write and len(set(zip(blocks, offsets))) != len(blocks):
        raise ValueError("duplicate KV write addresses in one traversal")
    return blocks, offsets


def build_kv_metadata(row_pages: Sequence[Sequence[int]], positions: Sequence[int], *,
                      block_size: int, device, sequence_keys=None, packed: bool = False,
                      for_write: bool = True) -> KVMetadata:
    """Plan and upload one traversal's metadata: one int64 and one int32 host
    buffer, each copied to the device once (as worker/buffers.py:153-199 stages
    them)."""
    positions = [int(p) for p in positions]
    blocks, offsets = write_addresses(row_pages, positions, block_size, for_write=for_write)
    plan = plan_attention_metadata(
        AttentionRows(block_tables=[tuple(p) for p in row_pages], positions=positions,
                      sequence_keys=sequence_keys if packed else None),
        block_size=block_size, packed_prefill=packed,
    )
    n, t, width = len(positions), plan.num_rows, plan.table_width
    device = torch.device(device)
    pin = device.type == "cuda"
    wide = torch.tensor(positions + blocks + offsets, dtype=torch.int64)
    narrow = torch.tensor(plan.block_tables + plan.context_lengths + (plan.cu_seqlens_q or []),
                          dtype=torch.int32)
    if pin:
        wide, narrow = wide.pin_memory(), narrow.pin_memory()
    wide = wide.to(device, non_blocking=pin)
    narrow = narrow.to(device, non_blocking=pin)
    return KVMetadata(
        position_ids=wide[:n],
        write_blocks=wide[n : 2 * n],
        write_offsets=wide[2 * n : 3 * n],
        block_tables=narrow[: t * width].view(t, width),
        context_lengths=narrow[t * width : t * width + t],
        writable=for_write,
        cu_seqlens_q=(narrow[t * width + t : t * width + 2 * t + 1]
                      if plan.cu_seqlens_q is not None else None),
        max_seqlen_q=plan.max_seqlen_q,
    )


def device_kv_metadata(*, position_ids, write_blocks, write_offsets, block_tables,
                       context_lengths, write_mask=None, active_rows=None,
                       device=None) -> DeviceKVMetadata:
    """Borrow GPU-owned metadata after checking shapes, dtypes and devices on
    the host (no device value is read)."""
    device = position_ids.device if device is None else torch.device(device)
    rows = position_ids.shape[0] if position_ids.ndim == 1 else -1
    for name, tensor, dtype in (("position_ids", position_ids, torch.int64),
                                ("write_blocks", write_blocks, torch.int64),
                                ("write_offsets", write_offsets, torch.int64),
                                ("context_lengths", context_lengths, torch.int32)):
        if tensor.shape != (rows,) or tensor.dtype != dtype or tensor.device != device:
            raise ValueError(f"{name} must have shape [rows] and use {dtype} on {device}")
    if (block_tables.ndim != 2 or block_tables.shape[0] != rows or block_tables.shape[1] == 0
            or block_tables.dtype != torch.int32 or block_tables.device != device
            or not block_tables.is_contiguous()):
        raise ValueError("device block tables must be contiguous int32 [rows, pages]")
    if write_mask is not None and (write_mask.shape != (rows,) or write_mask.dtype != torch.bool
                                   or write_mask.device != device):
        raise ValueError("write_mask must be bool [rows] on the metadata device")
    if active_rows is not None and (active_rows.dtype != torch.int32 or active_rows.numel() != 1
                                    or active_rows.device != device):
        raise ValueError("active_rows must be an int32 scalar on the metadata device")
    return DeviceKVMetadata(position_ids, write_blocks, write_offsets, block_tables,
                            context_lengths, write_mask, active_rows)
