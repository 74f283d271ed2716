"""Paged KV pool with LAST_EXITED or SHARED depth planes, on the hip kernels.

Host-side mirror of the reference's vllm_rlt/core/kv_cache_manager.py for the
hot-path operations (same method names, argument meaning and errors):

  pool            [num_blocks, num_layers, block_size, kv_heads, head_dim] K and V
                  (reference :143-145); a block holds every layer.
  planes          LAST_EXITED keeps one block table per loop depth, SHARED one
                  table for all depths (reference :525-526).
  allocate/free   refcounted pages, optional prefix reuse keyed by a SHA-256
                  chain of 16-token pages (reference :191-319).
  write           append, -> vrh_kv_append (reference :676-701)
  attend          decode / packed prefill / windowed, -> vrh_paged_decode,
                  vrh_paged_prefill (reference :712-803)
  finalize_token  depth propagation, -> vrh_kv_finalize_token (reference :806-831)
  read            history gather, -> vrh_kv_gather (reference :834-854)
  snapshot/restore preemption page copies to/from host (reference :481-523)
  copy_blocks     on-device whole-block copy, -> vrh_kv_copy_blocks (copy-on-write
                  and compaction; the reference has no on-device block copy)

Written-position bookkeeping (``_WrittenPositions``) guards attention against
reading KV that was never written, as in the reference (:31-50, :703-710).
All KV bytes move through the HIP library; this module never computes
attention or copies KV itself, except snapshot/restore's host transfers.
"""

from __future__ import annotations

import hashlib
import struct
from collections import OrderedDict
from collections.abc import Sequence
from copy import deepcopy
from dataclasses import dataclass, field
from numbers import Integral

import torch

from vllm_rlt.attention import (
    AttentionBackend,
    BackendCapabilities,
    backend_capabilities,
    create_backend,
    validate_backend_name,
)
from vllm_rlt.kernels import hip_attention as hip
from vllm_rlt.worker.metadata import DeviceKVMetadata, KVMetadata, MetadataBuilder


@dataclass
class _WrittenPositions:
    """Positions written for one (plane, layer): a dense prefix plus stragglers."""

    prefix: int = 0
    pending: set[int] = field(default_factory=set)

    def add(self, position: int) -> None:
        if position < self.prefix:
            return
        if position != self.prefix:
            self.pending.add(position)
            return
        self.prefix += 1
        while self.prefix in self.pending:
            self.pending.discard(self.prefix)
            self.prefix += 1

    def __contains__(self, position: int) -> bool:
        return position < self.prefix or position in self.pending


@dataclass
class _Allocation:
    max_tokens: int
    block_tables: tuple[tuple[int, ...], ...]
    written: list[list[_WrittenPositions]]


@dataclass(frozen=True)
class KVSnapshot:
    """A preempted request's pages (host, ``[pages * planes, L, bs, H, D]`` in
    block-table order) and its written state."""

    max_tokens: int
    pages: int
    written: list[list[_WrittenPositions]]
    keys: torch.Tensor
    values: torch.Tensor


def _positive(name, value):
    if not isinstance(value, Integral) or isinstance(value, bool) or value <= 0:
        raise ValueError(f"{name} must be a positive integer")
    return int(value)


class KVCacheManager:
    """Own a fixed physical page pool shared by request/depth allocations."""

    def __init__(
        self,
        num_layers: int,
        num_kv_heads: int,
        head_dim: int,
        num_blocks: int,
        block_size: int,
        max_loops: int,
        device: str | torch.device = "cuda",
        dtype: torch.dtype = torch.bfloat16,
        backend: str = "auto",
        layout: str = "last_exited",
        enable_prefix_caching: bool = False,
        recurrent_layers: Sequence[int] | None = None,
        *,
        attention: AttentionBackend | None = None,
    ):
        self.num_layers = _positive("num_layers", num_layers)
        self.num_kv_heads = _positive("num_kv_heads", num_kv_heads)
        self.head_dim = _positive("head_dim", head_dim)
        self.num_blocks = _positive("num_blocks", num_blocks)
        self.block_size = _positive("block_size", block_size)
        self.max_loops = _positive("max_loops", max_loops)
        validate_backend_name(backend)
        if dtype not in {torch.float32, torch.float16, torch.bfloat16}:
            raise ValueError("KV dtype must be float32, float16, or bfloat16")
        if layout not in {"last_exited", "shared"}:
            raise ValueError("unsupported KV layout")
        if enable_prefix_caching and layout != "last_exited":
            raise ValueError("prefix caching requires last_exited KV")
        self.layout = layout
        self.recurrent_layers = (
            tuple(range(num_layers)) if recurrent_layers is None else tuple(recurrent_layers)
        )
        if not self.recurrent_layers or len(set(self.recurrent_layers)) != len(
            self.recurrent_layers
        ):
            raise ValueError("recurrent_layers must be nonempty and unique")
        if any(type(x) is not int or not 0 <= x < num_layers for x in self.recurrent_layers):
            raise ValueError("recurrent_layers must be valid cache layer indices")
        self.storage_depths = max_loops if layout == "last_exited" else 1
        self.device = torch.device(device)
        self.dtype = dtype
        self.attention = attention or create_backend(
            backend, self.device, dtype, head_dim, block_size
        )
        self.attention_info = self.attention.info
        self.backend = self.attention_info.get("selected_backend", "hip")
        shape = (num_blocks, num_layers, block_size, num_kv_heads, head_dim)
        self.key_cache = torch.empty(shape, device=self.device, dtype=dtype)
        self.value_cache = torch.empty_like(self.key_cache)
        self.device = self.key_cache.device
        self._free_blocks = list(reversed(range(num_blocks)))
        self._allocations: dict[str, _Allocation] = {}
        self._refs = [0] * num_blocks
        self._prefixes: OrderedDict[bytes, tuple[int, ...]] = OrderedDict()
        self.enable_prefix_caching = enable_prefix_caching
        self.prefix_hits = self.prefix_queries = 0

    # ------------------------------------------------------------ capacity
    @property
    def attention_capabilities(self) -> BackendCapabilities:
        return backend_capabilities(self.attention)

    @property
    def num_free_blocks(self) -> int:
        cached_only = sum(self._refs[b] == 1 for blocks in self._prefixes.values() for b in blocks)
        return len(self._free_blocks) + cached_only

    @property
    def num_used_blocks(self) -> int:
        return self.num_blocks - self.num_free_blocks

    @property
    def bytes_per_block(self) -> int:
        return (2 * self.num_layers * self.block_size * self.num_kv_heads * self.head_dim
                * self.key_cache.element_size())

    def required_blocks(self, max_tokens: int) -> int:
        if not isinstance(max_tokens, Integral) or isinstance(max_tokens, bool) or max_tokens <= 0:
            raise ValueError("max_tokens must be a positive integer")
        return -(-max_tokens // self.block_size) * self.storage_depths

    def _drop_refs(self, blocks):
        for b in blocks:
            self._refs[b] -= 1
            assert self._refs[b] >= 0
            if self._refs[b] == 0:
                self._free_blocks.append(b)

    def _claim(self, count):
        """Take ``count`` blocks, evicting cached prefixes only if that suffices."""
        if len(self._free_blocks) < count and self.num_free_blocks < count:
            return None
        while len(self._free_blocks) < count and self._prefixes:
            _, blocks = self._prefixes.popitem(last=False)
            self._drop_refs(blocks)
        if len(self._free_blocks) < count:
            return None
        blocks = [self._free_blocks.pop() for _ in range(count)]
        for b in blocks:
            self._refs[b] = 1
        return blocks

    # -------------------------------------------------------------- prefix
    def _prefix_keys(self, tokens):
        digest = b""
        full = len(tokens) // self.block_size * self.block_size
        for start in range(0, full, self.block_size):
            page = tokens[start : start + self.block_size]
            digest = hashlib.sha256(digest + struct.pack(f"<{len(page)}q", *page)).digest()
            yield digest

    def publish_prefix(self, request_id, tokens, length):
        """Index complete, fully written prompt pages for zero-copy reuse."""
        if not self.enable_prefix_caching:
            return
        allocation = self._get_allocation(request_id)
        pages = min(length, len(tokens) - 1) // self.block_size
        for index, key in enumerate(self._prefix_keys(tokens[: pages * self.block_size])):
            if key in self._prefixes:
                self._prefixes.move_to_end(key)
                continue
            blocks = tuple(table[index] for table in allocation.block_tables)
            for b in blocks:
                self._refs[b] += 1
            self._prefixes[key] = blocks

    def lookup_prefix(self, tokens):
        if not self.enable_prefix_caching:
            return ()
        found = []
        for key in self._prefix_keys(tokens[:-1]):
            blocks = self._prefixes.get(key)
            if blocks is None:
                break
            self._prefixes.move_to_end(key)
            found.append(blocks)
        return tuple(found)

    def exclusive_prefix_blocks(self, prefix) -> int:
        return sum(self._refs[b] == 1 for group in prefix for b in group)

    # ---------------------------------------------------------- allocation
    def allocate(self, request_id: str, max_tokens: int, *, prefix=()) -> bool:
        if not isinstance(request_id, str) or not request_id:
            raise ValueError("request_id must be a nonempty string")
        if request_id in self._allocations:
            raise ValueError(f"request {request_id!r} already owns KV blocks")
        required = self.required_blocks(max_tokens)
        if required > self.num_blocks:
            raise ValueError(
                f"request needs {required} physical KV blocks, but the pool has {self.num_blocks}"
            )
        pages = -(-max_tokens // self.block_size)
        if len(prefix) > pages:
            raise ValueError("prefix exceeds the request's pages")
        shared = [b for group in prefix for b in group]
        for b in shared:
            self._refs[b] += 1
        tail = pages - len(prefix)
        fresh = self._claim(tail * self.storage_depths)
        if fresh is None:
            self._drop_refs(shared)
            return False
        tables = tuple(
            tuple(group[d] for group in prefix) + tuple(fresh[d * tail : (d + 1) * tail])
            for d in range(self.storage_depths)
        )
        done = len(prefix) * self.block_size
        self._allocations[request_id] = _Allocation(
            int(max_tokens),
            tables,
            [[_WrittenPositions(prefix=done) for _ in range(self.num_layers)]
             for _ in range(self.storage_depths)],
        )
        self.prefix_queries += 1
        self.prefix_hits += done
        return True

    def free(self, request_id: str) -> None:
        allocation = self._allocations.pop(request_id, None)
        if allocation is not None:
            self._drop_refs(b for table in allocation.block_tables for b in reversed(table))

    def has_allocation(self, request_id: str) -> bool:
        return request_id in self._allocations

    def allocated_blocks(self, request_id: str) -> int:
        return len(self._get_allocation(request_id).block_tables[0]) * self.storage_depths

    def get_block_table(self, request_id: str, depth: int) -> tuple[int, ...]:
        self._validate_depth(depth)
        return self._get_allocation(request_id).block_tables[self._plane(depth)]

    def plane_block_tables(self, request_id: str) -> tuple[tuple[int, ...], ...]:
        return self._get_allocation(request_id).block_tables

    def _plane(self, depth: int) -> int:
        return depth if self.layout == "last_exited" else 0

    def _get_allocation(self, request_id: str) -> _Allocation:
        try:
            return self._allocations[request_id]
        except KeyError:
            raise KeyError(f"request {request_id!r} has no KV allocation") from None

    # ---------------------------------------------------------- validation
    def _validate_layer(self, layer: int) -> None:
        if not isinstance(layer, Integral) or isinstance(layer, bool) or not (
            0 <= layer < self.num_layers
        ):
            raise ValueError(f"layer must be in [0, {self.num_layers})")

    def _validate_depth(self, depth: int) -> None:
        if not isinstance(depth, Integral) or isinstance(depth, bool) or not (
            0 <= depth < self.max_loops
        ):
            raise ValueError(f"depth must be in [0, {self.max_loops})")

    def _validate_position(self, allocation: _Allocation, position: int) -> None:
        if not isinstance(position, Integral) or isinstance(position, bool) or not (
            0 <= position < allocation.max_tokens
        ):
            raise ValueError(f"position must be in [0, {allocation.max_tokens})")

    def _validate_rows(self, request_ids, depths, positions):
        if isinstance(positions, torch.Tensor):
            if positions.ndim != 1 or positions.dtype not in {torch.int32, torch.int64}:
                raise ValueError("positions must be a one-dimensional integer tensor")
            positions = positions.tolist()
        if len(request_ids) != len(depths) or len(request_ids) != len(positions):
            raise ValueError("request_ids, depths, and positions must have equal lengths")
        rows = []
        for request_id, depth, position in zip(request_ids, depths, positions):
            allocation = self._get_allocation(request_id)
            self._validate_depth(depth)
            self._validate_position(allocation, position)
            rows.append((allocation, int(depth), int(position)))
        return rows

    def _validate_tensor(self, tensor, batch_size, name, *, query=False):
        if tensor.ndim != 3 or tensor.shape[0] != batch_size or tensor.shape[-1] != self.head_dim:
            raise ValueError(f"{name} must have shape [batch, heads, {self.head_dim}]")
        if query:
            if tensor.shape[1] == 0 or tensor.shape[1] % self.num_kv_heads:
                raise ValueError("query heads must be a positive multiple of KV heads")
        elif tensor.shape[1] != self.num_kv_heads:
            raise ValueError(f"{name} must have {self.num_kv_heads} KV heads")
        if tensor.device != self.device or tensor.dtype != self.dtype:
            raise ValueError(f"{name} must use device {self.device} and dtype {self.dtype}")

    def _require_live_batch(self, batch) -> None:
        if isinstance(batch, KVMetadata) and batch.owner is not self:
            raise ValueError("prepared KV batch belongs to a different cache manager")
        for request_id, allocation in batch.allocations:
            if self._allocations.get(request_id) is not allocation:
                raise RuntimeError(f"stale prepared KV batch for request {request_id!r}")

    def _require_prefix(self, allocation, layer, depth, length):
        if length > allocation.written[self._plane(depth)][layer].prefix:
            raise RuntimeError(
                f"uninitialized KV history at layer {layer}, depth {depth}, "
                f"context length {length}; "
                "write preceding tokens and finalize early exits before attention"
            )

    # ------------------------------------------------------------ metadata
    @property
    def metadata_builder(self) -> MetadataBuilder:
        return MetadataBuilder(self)

    def _stage(self, values, dtype):
        host = torch.tensor(values, dtype=dtype, pin_memory=self.device.type == "cuda")
        return host.to(self.device, non_blocking=True)

    def _prepare_batch(self, request_ids, depths, positions, *, for_write=True,
                       packed_prefill=False) -> KVMetadata:
        return self.metadata_builder.build(
            request_ids, depths, positions, packed=packed_prefill, for_write=for_write
        )

    # --------------------------------------------------------------- write
    @torch.no_grad()
    def write(self, layer, request_ids, depths, positions, k, v) -> None:
        """Append a batch's K/V at each row's (depth plane, position)."""
        self._validate_layer(layer)
        batch = self._prepare_batch(request_ids, depths, positions)
        self._write_prepared(layer, batch, k, v)

    @torch.no_grad()
    def _write_prepared(self, layer, batch, k, v) -> None:
        self._validate_layer(layer)
        self._require_live_batch(batch)
        rows = len(batch.position_ids)
        self._validate_tensor(k, rows, "k")
        self._validate_tensor(v, rows, "v")
        if isinstance(batch, DeviceKVMetadata):
            hip.kv_append(
                self.key_cache[:, layer], self.value_cache[:, layer], k, v, batch.write_blocks,
                batch.write_offsets, write_mask=batch.write_mask, active_rows=batch.active_rows,
            )
            return
        if not batch.writable:
            raise ValueError("a read-only prepared KV batch cannot be written")
        if not batch.rows:
            return
        n = len(batch.rows)
        hip.kv_append(
            self.key_cache[:, layer], self.value_cache[:, layer], k[:n], v[:n],
            batch.write_blocks, batch.write_offsets,
        )
        for allocation, depth, position in batch.rows:
            allocation.written[self._plane(depth)][layer].add(position)

    # -------------------------------------------------------------- attend
    @torch.no_grad()
    def attend(self, layer, request_ids, depths, positions, q, *, window=None) -> torch.Tensor:
        """Causal attention of each row at its own position and depth plane."""
        self._validate_layer(layer)
        batch = self._prepare_batch(request_ids, depths, positions, for_write=False)
        return self._attend_prepared(layer, batch, q, window=window)

    def prepare(self, request_ids, depths, positions, *, packed=False,
                for_write=True) -> KVMetadata:
        """Build one traversal's metadata (reference ``prepare_recurrent``); with
        ``packed`` contiguous (request, depth) runs become prefill sequences."""
        return self._prepare_batch(
            request_ids, depths, positions, for_write=for_write,
            packed_prefill=packed and self.attention_capabilities.packed_prefill,
        )

    @torch.no_grad()
    def _attend_prepared(self, layer, batch, q, *, window=None) -> torch.Tensor:
        self._validate_layer(layer)
        self._require_live_batch(batch)
        self._validate_tensor(q, len(batch.position_ids), "q", query=True)
        if window is not None:
            return self._attend_windowed(layer, batch, q, window)
        kc, vc = self.key_cache[:, layer], self.value_cache[:, layer]
        if isinstance(batch, DeviceKVMetadata):
            return self.attention(q, kc, vc, batch.block_tables, batch.context_lengths)
        if not batch.rows:
            return torch.empty_like(q)
        for allocation, depth, position in batch.rows:
            self._require_prefix(allocation, layer, depth, position + 1)
        if batch.cu_seqlens_q is not None:
            return self.attention.prefill(q, kc, vc, batch.block_tables, batch.context_lengths,
                                          batch.cu_seqlens_q, batch.max_seqlen_q)
        return self.attention(q, kc, vc, batch.block_tables, batch.context_lengths)

    @torch.no_grad()
    def _attend_windowed(self, layer, batch, q, window) -> torch.Tensor:
        if isinstance(window, bool) or not isinstance(window, int) or window <= 0:
            raise ValueError("window must be a positive integer")
        if not self.attention_capabilities.sliding_window:
            raise NotImplementedError(
                f"the {self.backend} attention backend does not implement sliding-window masking"
            )
        if batch.cu_seqlens_q is not None:
            raise NotImplementedError("sliding-window attention needs one query row per token")
        if not isinstance(batch, DeviceKVMetadata):
            if not batch.rows:
                return torch.empty_like(q)
            for allocation, depth, position in batch.rows:
                self._require_prefix(allocation, layer, depth, position + 1)
        return self.attention.windowed(q, self.key_cache[:, layer], self.value_cache[:, layer],
                                       batch.block_tables, batch.context_lengths, window)

    # ------------------------------------------------------------ finalize
    def token_written(self, request_id: str, position: int, depth: int) -> bool:
        allocation = self._get_allocation(request_id)
        self._validate_depth(depth)
        self._validate_position(allocation, position)
        plane = allocation.written[self._plane(depth)]
        return all(position in plane[layer] for layer in range(self.num_layers))

    def exit_written(self, request_id: str, position: int, depth: int) -> bool:
        allocation = self._get_allocation(request_id)
        self._validate_depth(depth)
        self._validate_position(allocation, position)
        plane = allocation.written[self._plane(depth)]
        return all(position in plane[layer] for layer in self.recurrent_layers)

    def _require_exit_written(self, request_id, position, exit_depth) -> _Allocation:
        allocation = self._get_allocation(request_id)
        self._validate_depth(exit_depth)
        self._validate_position(allocation, position)
        plane = allocation.written[self._plane(exit_depth)]
        if any(position not in plane[layer] for layer in self.recurrent_layers):
            raise RuntimeError(
                "cannot finalize a token before every layer has written its exit depth"
            )
        return allocation

    def _record_finalized(self, allocation, position, exit_depth) -> None:
        if self.layout == "shared":
            return
        for depth in range(exit_depth + 1, self.max_loops):
            for layer in self.recurrent_layers:
                allocation.written[self._plane(depth)][layer].add(position)

    def mark_finalized(self, request_id: str, position: int, exit_depth: int) -> None:
        """Bookkeeping half of ``finalize_token`` (after a device-side copy)."""
        allocation = self._require_exit_written(request_id, position, exit_depth)
        self._record_finalized(allocation, position, exit_depth)

    @torch.no_grad()
    def finalize_token(self, request_id: str, position: int, exit_depth: int) -> None:
        """Propagate the exit depth's K/V into every deeper (unexecuted) plane."""
        allocation = self._require_exit_written(request_id, position, exit_depth)
        if self.layout == "shared":
            return
        page, offset = divmod(position, self.block_size)
        source = allocation.block_tables[self._plane(exit_depth)][page]
        targets = [allocation.block_tables[self._plane(d)][page]
                   for d in range(exit_depth + 1, self.max_loops)]
        hip.kv_finalize_token(self.key_cache, self.value_cache, source, targets, offset,
                              self.recurrent_layers)
        self._record_finalized(allocation, position, exit_depth)

    # ---------------------------------------------------------------- read
    @torch.no_grad()
    def read(self, layer: int, request_id: str, depth: int, length: int | None = None):
        """Materialise a fully written prefix as ``[token, kv_head, dim]`` K and V."""
        self._validate_layer(layer)
        self._validate_depth(depth)
        allocation = self._get_allocation(request_id)
        if length is None:
            length = allocation.written[self._plane(depth)][layer].prefix
        if not isinstance(length, Integral) or isinstance(length, bool) or not (
            0 <= length <= allocation.max_tokens
        ):
            raise ValueError("read length exceeds the request's reserved token budget")
        self._require_prefix(allocation, layer, depth, length)
        table = torch.tensor(allocation.block_tables[self._plane(depth)], dtype=torch.int32)
        return hip.kv_gather(self.key_cache[:, layer], self.value_cache[:, layer],
                             table.to(self.device), length)

    # ------------------------------------------------------ block movement
    @torch.no_grad()
    def copy_blocks(self, src_blocks: Sequence[int], dst_blocks: Sequence[int]) -> None:
        """Copy whole physical blocks (every layer, K and V) on the device."""
        if len(src_blocks) != len(dst_blocks):
            raise ValueError("src_blocks and dst_blocks must have equal lengths")
        for b in (*src_blocks, *dst_blocks):
            if not isinstance(b, Integral) or not 0 <= b < self.num_blocks:
                raise ValueError("block id out of range")
        if set(src_blocks) & set(dst_blocks) or len(set(dst_blocks)) != len(dst_blocks):
            raise ValueError("copy destinations must be distinct and disjoint from sources")
        if not src_blocks:
            return
        index = self._stage(list(src_blocks) + list(dst_blocks), torch.int64)
        n = len(src_blocks)
        hip.kv_copy_blocks(self.key_cache, self.value_cache, index[:n], index[n:])

    def snapshot(self, request_id: str) -> KVSnapshot:
        """Copy a request's pages and written state to the host.

        Reference: core/kv_cache_manager.py:481-502. Instead of one copy per
        page, a single kernel writes every page straight into pinned host rows
        (no device staging buffer, the reference's reason for copying page by
        page). Returns once the host rows are complete.
        """
        allocation = self._get_allocation(request_id)
        blocks = [b for table in allocation.block_tables for b in table]
        if self.device.type != "cuda":
            raise ValueError("snapshot of the hip build needs a ROCm device pool")
        keys = torch.empty((len(blocks), *self.key_cache.shape[1:]), dtype=self.dtype,
                           pin_memory=True)
        values = torch.empty_like(keys, pin_memory=True)
        index = torch.tensor(blocks, dtype=torch.int64).to(self.device)
        hip.kv_blocks_to_host(self.key_cache, self.value_cache, index, keys, values)
        torch.cuda.current_stream(self.device).synchronize()
        return KVSnapshot(allocation.max_tokens, len(allocation.block_tables[0]),
                          deepcopy(allocation.written), keys, values)

    def restore(self, request_id: str, snapshot: KVSnapshot) -> None:
        """Load a snapshot into a fresh allocation of the same size.

        Reference: core/kv_cache_manager.py:504-523. One kernel reads the
        snapshot's host rows into the new blocks on the current stream; the
        call returns after that stream has finished with the host rows, so the
        caller may drop the snapshot immediately (the reference's host copies
        are blocking too).
        """
        allocation = self._get_allocation(request_id)
        if allocation.max_tokens != snapshot.max_tokens:
            raise ValueError("snapshot capacity does not match the allocation")
        if len(allocation.block_tables[0]) != snapshot.pages:
            raise ValueError("snapshot page count does not match the allocation")
        if any(w.prefix or w.pending for plane in allocation.written for w in plane):
            raise RuntimeError("cannot restore into an allocation that already holds KV")
        blocks = [b for table in allocation.block_tables for b in table]
        if self.device.type != "cuda":
            raise ValueError("restore of the hip build needs a ROCm device pool")
        keys, values = snapshot.keys, snapshot.values
        if not keys.is_pinned():
            keys, values = keys.pin_memory(), values.pin_memory()
        index = torch.tensor(blocks, dtype=torch.int64).to(self.device)
        hip.kv_blocks_from_host(self.key_cache, self.value_cache, index, keys, values)
        torch.cuda.current_stream(self.device).synchronize()
        allocation.written = deepcopy(snapshot.written)
