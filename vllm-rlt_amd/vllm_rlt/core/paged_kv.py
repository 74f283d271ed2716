"""The device half of a depth-aware paged KV cache: the pool and its hot-path
operations, addressed by physical pages.

The reference keeps its request bookkeeping (allocator, refcounts, prefix
cache, written-position tracking) in vllm_rlt/core/kv_cache_manager.py, and
that manager stays as it is. What it does to KV *bytes* is what this class
does on gfx950, given the physical pages the manager resolved:

  pool            ``[num_blocks, num_layers, block_size, kv_heads, head_dim]``
                  K and V (reference kv_cache_manager.py:143-145); a block
                  holds every layer, so block copies move contiguous bytes
  append          kv_cache_manager.py:676-701 (``_write_prepared``), the
                  masked / bucketed forms of kernels/routing.py:180-225 and
                  kernels/graph_kv.py:7-65 -> vrh_kv_append
  attend/prefill  kv_cache_manager.py:729-803 -> vrh_paged_decode,
                  vrh_paged_prefill (via the attention backend)
  finalize_token  kv_cache_manager.py:806-831 -> vrh_kv_finalize_token
  finalize        kernels/routing.py:147-177 -> vrh_kv_finalize
  read            kv_cache_manager.py:834-854 -> vrh_kv_gather
  snapshot/restore kv_cache_manager.py:481-523 -> vrh_kv_blocks_to_host /
                  vrh_kv_blocks_from_host (one launch per direction)
  copy_blocks     whole-block copy -> vrh_kv_copy_blocks (copy-on-write of a
                  shared page, compaction; no reference counterpart)

Pages are plain block ids. A request's LAST_EXITED layout is one page list
per loop depth ("plane"); SHARED is one list for every depth. Which pages a
request owns, and whether a position was written, is the caller's business:
nothing here allocates pages or tracks writes.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass
from numbers import Integral

import torch

from vllm_rlt.kernels import hip_attention as hip


def _count(name: str, value) -> int:
    if not isinstance(value, Integral) or isinstance(value, bool) or value <= 0:
        raise ValueError(f"{name} must be a positive integer")
    return int(value)


@dataclass(frozen=True)
class PageSnapshot:
    """Pages copied to pinned host memory: row i is page i of the list given
    to :meth:`PagedKVPool.snapshot`, ``[pages, L, bs, H, D]`` per K and V."""

    keys: torch.Tensor
    values: torch.Tensor

    @property
    def pages(self) -> int:
        return self.keys.shape[0]


class PagedKVPool:
    """K/V page pool on one ROCm device plus the operations that move its bytes."""

    def __init__(self, num_blocks, num_layers, block_size, num_kv_heads, head_dim, *,
                 dtype=torch.bfloat16, device="cuda", attention=None):
        shape = (_count("num_blocks", num_blocks), _count("num_layers", num_layers),
                 _count("block_size", block_size), _count("num_kv_heads", num_kv_heads),
                 _count("head_dim", head_dim))
        hip.dtype_code(dtype)
        self.device = torch.device(device)
        self.dtype = dtype
        self.num_blocks, self.num_layers, self.block_size = shape[:3]
        self.num_kv_heads, self.head_dim = shape[3:]
        # Zero-filled, so a page that was never written reads as zeros.
        self.key_cache = torch.zeros(shape, dtype=dtype, device=self.device)
        self.value_cache = torch.zeros_like(self.key_cache)
        self._attention = attention

    # ------------------------------------------------------------- helpers
    @property
    def attention(self):
        """The attention backend (``create_backend('hip', ...)`` on first use)."""
        if self._attention is None:
            from vllm_rlt.attention import create_backend

            self._attention = create_backend("hip", self.device, self.dtype, self.head_dim,
                                             self.block_size)
        return self._attention

    def layer(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The ``[blocks, block_size, kv_heads, head_dim]`` views of one layer."""
        if isinstance(layer, bool) or not isinstance(layer, Integral) \
                or not 0 <= layer < self.num_layers:
            raise ValueError(f"layer must be in [0, {self.num_layers})")
        return self.key_cache[:, layer], self.value_cache[:, layer]

    def _pages(self, name: str, pages) -> list[int]:
        values = pages.tolist() if isinstance(pages, torch.Tensor) else list(pages)
        out = []
        for page in values:
            if isinstance(page, bool) or not isinstance(page, Integral):
                raise ValueError(f"{name} must hold integer block ids")
            if not 0 <= page < self.num_blocks:
                raise ValueError(f"{name}: block {page} out of range [0, {self.num_blocks})")
            out.append(int(page))
        return out

    def _index(self, pages: list[int]) -> torch.Tensor:
        return torch.tensor(pages, dtype=torch.int64, device=self.device)

    # -------------------------------------------------------------- writes
    def append(self, layer, k, v, write_blocks, write_offsets, *, write_mask=None,
               active_rows=None) -> None:
        """``K[write_blocks[r], layer, write_offsets[r]] = k[r]`` (and V) for the
        enabled rows (``write_mask``, ``r < active_rows``); bit-exact."""
        key_cache, value_cache = self.layer(layer)
        hip.kv_append(key_cache, value_cache, k, v, write_blocks, write_offsets,
                      write_mask=write_mask, active_rows=active_rows)

    def append_layers(self, first_layer, k, v, write_blocks, write_offsets, *,
                      write_mask=None) -> None:
        """One launch for ``k, v : [layers, rows, H, D]`` into consecutive layers."""
        self.layer(first_layer)
        hip.kv_append_layers(self.key_cache, self.value_cache, first_layer, k, v, write_blocks,
                             write_offsets, write_mask=write_mask)

    # ------------------------------------------------------------ attention
    def attend(self, layer, q, block_tables, context_lengths, *, window=None) -> torch.Tensor:
        """Single-query paged attention of one layer (``window``: last keys only)."""
        key_cache, value_cache = self.layer(layer)
        if window is None:
            return self.attention(q, key_cache, value_cache, block_tables, context_lengths)
        return self.attention.windowed(q, key_cache, value_cache, block_tables, context_lengths,
                                       window)

    def prefill(self, layer, q, block_tables, context_lengths, cu_seqlens_q,
                max_seqlen_q) -> torch.Tensor:
        """Packed causal prefill of one layer, bottom-right aligned per sequence."""
        key_cache, value_cache = self.layer(layer)
        return self.attention.prefill(q, key_cache, value_cache, block_tables, context_lengths,
                                      cu_seqlens_q, max_seqlen_q)

    def read(self, layer, pages, length) -> tuple[torch.Tensor, torch.Tensor]:
        """The first ``length`` tokens of a page list as ``[length, H, D]`` K and V."""
        key_cache, value_cache = self.layer(layer)
        pages = self._pages("pages", pages)
        if isinstance(length, bool) or not isinstance(length, Integral) \
                or not 0 <= length <= len(pages) * self.block_size:
            raise ValueError("length must be in [0, pages * block_size]")
        table = torch.tensor(pages or [0], dtype=torch.int32, device=self.device)
        return hip.kv_gather(key_cache, value_cache, table, int(length))

    # -------------------------------------------------------------- depths
    def finalize_token(self, plane_pages: Sequence[Sequence[int]], position: int,
                       exit_depth: int, layers: Sequence[int] | None = None) -> None:
        """LAST_EXITED: position ``position`` exited at ``exit_depth``; copy its
        K/V slot (every layer, or ``layers``) from that depth's page into the
        same slot of every deeper plane. One plane (SHARED) copies nothing."""
        planes = len(plane_pages)
        if not 0 <= exit_depth < planes:
            raise ValueError(f"exit_depth must be in [0, {planes})")
        if position < 0:
            raise ValueError("position must be nonnegative")
        page = position // self.block_size
        if any(page >= len(p) for p in plane_pages):
            raise ValueError("position beyond a plane's pages")
        targets = self._pages("plane pages", [plane_pages[d][page]
                                               for d in range(exit_depth + 1, planes)])
        layers = list(range(self.num_layers)) if layers is None else list(layers)
        if any(not 0 <= layer < self.num_layers for layer in layers):
            raise ValueError(f"layers must be in [0, {self.num_layers})")
        if not targets or not layers:
            return
        source = self._pages("plane pages", [plane_pages[exit_depth][page]])[0]
        hip.kv_finalize_token(self.key_cache, self.value_cache, source, targets,
                              position % self.block_size, layers)

    def finalize(self, descriptors, tables, planes: int) -> None:
        """Device rows ``(slot, depth, position)`` over ``tables [slots * planes,
        width]``: the stream-ordered form of :meth:`finalize_token`."""
        hip.kv_finalize(self.key_cache, self.value_cache, descriptors, tables, planes)

    # --------------------------------------------------------- block moves
    def copy_blocks(self, src_blocks, dst_blocks) -> None:
        """``pool[dst[i]] = pool[src[i]]`` for whole blocks of K and V."""
        src, dst = self._pages("src_blocks", src_blocks), self._pages("dst_blocks", dst_blocks)
        if len(src) != len(dst):
            raise ValueError("src_blocks and dst_blocks must have equal lengths")
        if len(set(dst)) != len(dst) or set(src) & set(dst):
            raise ValueError("destination blocks must be distinct and disjoint from the sources")
        if src:
            hip.kv_copy_blocks(self.key_cache, self.value_cache, self._index(src),
                               self._index(dst))

    def snapshot(self, pages) -> PageSnapshot:
        """Copy pages (all layers, K and V) to pinned host rows in list order;
        returns once the copies are complete."""
        pages = self._pages("pages", pages)
        shape = (len(pages), *self.key_cache.shape[1:])
        keys = torch.empty(shape, dtype=self.dtype, pin_memory=True)
        values = torch.empty(shape, dtype=self.dtype, pin_memory=True)
        if pages:
            hip.kv_blocks_to_host(self.key_cache, self.value_cache, self._index(pages), keys,
                                  values)
            torch.cuda.current_stream(self.device).synchronize()
        return PageSnapshot(keys, values)

    def restore(self, pages, snapshot: PageSnapshot) -> None:
        """Copy a snapshot's rows into ``pages`` (which may differ from the pages
        it was taken from); refused unless the page counts match."""
        pages = self._pages("pages", pages)
        if len(pages) != snapshot.pages:
            raise ValueError(f"snapshot page count {snapshot.pages} differs from the "
                             f"{len(pages)} target pages")
        if len(set(pages)) != len(pages):
            raise ValueError("restore target pages must be distinct")
        if pages:
            hip.kv_blocks_from_host(self.key_cache, self.value_cache, self._index(pages),
                                    snapshot.keys, snapshot.values)
            torch.cuda.current_stream(self.device).synchronize()
