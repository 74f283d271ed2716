"""Kernel metadata planning: depth-selected page tables and causal lengths.

Same contract as the reference's vllm_rlt/attention/metadata.py:23-121:
  * one table row per query row, padded with -1 to the batch's width
    ``max(position // block_size + 1)``; length = position + 1;
  * packed prefill groups runs of equal ``sequence_keys`` (contiguous
    positions, each key one run) into sequences with ``cu_seqlens_q``; the
    sequence's table row and length come from its last query row.
Tables and lengths are int32 (the dtypes the hip kernels consume).
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class AttentionRows:
    """One traversal after each row's physical depth plane has been selected."""

    block_tables: Sequence[tuple[int, ...]]
    positions: Sequence[int]
    sequence_keys: Sequence[tuple[object, int]] | None = None


@dataclass(frozen=True)
class AttentionMetadata:
    """Kernel-ready tensors borrowed for one execution traversal."""

    block_tables: torch.Tensor
    context_lengths: torch.Tensor
    cu_seqlens_q: torch.Tensor | None
    max_seqlen_q: int


@dataclass(frozen=True)
class AttentionMetadataValues:
    """Host values, staged by the caller into its own buffers."""

    block_tables: list[int]
    num_rows: int
    table_width: int
    context_lengths: list[int]
    cu_seqlens_q: list[int] | None
    max_seqlen_q: int


def _packed_runs(rows: AttentionRows) -> tuple[list[int], list[int]]:
    """Last row index of each sequence and the cumulative query counts."""
    keys, positions = rows.sequence_keys, rows.positions
    last_rows: list[int] = []
    cumulative = [0]
    seen = set()
    for index, key in enumerate(keys):
        continues = index > 0 and key == keys[index - 1]
        if continues:
            if positions[index] != positions[index - 1] + 1:
                raise ValueError("packed prefill positions must be contiguous")
            last_rows[-1] = index
            cumulative[-1] = index + 1
            continue
        if key in seen:
            raise ValueError("packed prefill request/depth must form one sequence")
        seen.add(key)
        last_rows.append(index)
        cumulative.append(index + 1)
    return last_rows, cumulative


def plan_attention_metadata(
    rows: AttentionRows,
    *,
    block_size: int,
    packed_prefill: bool = False,
) -> AttentionMetadataValues:
    """Pack selected tables and causal lengths without touching KV ownership."""
    if len(rows.block_tables) != len(rows.positions):
        raise ValueError("attention tables and positions must have equal lengths")
    if packed_prefill and rows.sequence_keys is not None:
        if len(rows.sequence_keys) != len(rows.positions):
            raise ValueError("packed attention keys and positions must have equal lengths")
    width = max((p // block_size + 1 for p in rows.positions), default=0)
    selected: Sequence[int] = range(len(rows.positions))
    cumulative = None
    max_query = 1
    if packed_prefill:
        if rows.sequence_keys is None:
            raise ValueError("packed prefill requires sequence keys")
        selected, cumulative = _packed_runs(rows)
        max_query = max((b - a for a, b in zip(cumulative, cumulative[1:])), default=1)
    tables: list[int] = []
    for index in selected:
        row = list(rows.block_tables[index][:width])
        tables.extend(row + [-1] * (width - len(row)))
    return AttentionMetadataValues(
        block_tables=tables,
        num_rows=len(selected),
        table_width=width,
        context_lengths=[rows.positions[index] + 1 for index in selected],
        cu_seqlens_q=cumulative,
        max_seqlen_q=max_query,
    )


def build_attention_metadata(
    rows: AttentionRows,
    *,
    block_size: int,
    device: torch.device,
    packed_prefill: bool = False,
) -> AttentionMetadata:
    """Materialise a plan for callers without a shared staging buffer."""
    plan = plan_attention_metadata(rows, block_size=block_size, packed_prefill=packed_prefill)
    tables = torch.tensor(plan.block_tables, dtype=torch.int32)
    return AttentionMetadata(
        block_tables=tables.reshape(plan.num_rows, plan.table_width).to(device),
        context_lengths=torch.tensor(plan.context_lengths, dtype=torch.int32).to(device),
        cu_seqlens_q=(
            torch.tensor(plan.cu_seqlens_q, dtype=torch.int32).to(device)
            if plan.cu_seqlens_q is not None
            else None
        ),
        max_seqlen_q=plan.max_seqlen_q,
    )
