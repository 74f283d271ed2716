"""PyTorch-facing adapter of the gfx950 paged-KV library (the ``hip`` backend).

Every function validates shapes/dtypes on the host (``ValueError``), passes raw
device pointers, element strides and the *current* HIP stream of the tensors'
device to the C ABI, and allocates outputs/workspace with PyTorch's caching
allocator (so HIP-graph capture owns them). Nothing here synchronises or reads
device values on the host.

Reference operator contracts mirrored here:
  HipPagedAttention.__call__  kernels/paged_attention.py:12-36,116-128
  HipPagedAttention.windowed  kernels/paged_attention.py:39-71
  HipPagedAttention.prefill   kernels/triton_attention.py:313-366
  kv_append                   core/kv_cache_manager.py:689-699,
                              kernels/routing.py:208-225, kernels/graph_kv.py:49-65
  kv_gather                   core/kv_cache_manager.py:834-854
  kv_finalize                 kernels/routing.py:147-177 + worker/model_runner.py:1331-1346
  kv_finalize_token           core/kv_cache_manager.py:806-831
  kv_copy_blocks              on-device block copy (copy-on-write; no reference counterpart)
  kv_blocks_to_host / kv_blocks_from_host
                              core/kv_cache_manager.py:481-523 (snapshot/restore copies)
  expand_kv_addresses         kernels/metadata.py:7-24
  routing_metadata / slots    kernels/routing.py:7-48
"""

from __future__ import annotations

import torch

from vllm_rlt.kernels._hip import VRH_DTYPE_BF16, VRH_DTYPE_F16, VRH_DTYPE_F32, library

_DTYPE_CODES = {
    torch.float32: VRH_DTYPE_F32,
    torch.float16: VRH_DTYPE_F16,
    torch.bfloat16: VRH_DTYPE_BF16,
}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"the hip backend supports float32, float16 and bfloat16, not {dtype}") \
            from None


def _stream(tensor: torch.Tensor) -> int:
    return torch.cuda.current_stream(tensor.device).cuda_stream


def _on_gpu(name: str, tensor: torch.Tensor, device: torch.device) -> None:
    if tensor.device.type != "cuda":
        raise ValueError(f"{name} must be a ROCm device tensor for the hip backend")
    if tensor.device != device:
        raise ValueError(f"{name} is on {tensor.device}, expected {device}")


def _check_int(name, tensor, dtype, ndim, device):
    _on_gpu(name, tensor, device)
    if tensor.dtype != dtype or tensor.ndim != ndim:
        raise ValueError(f"{name} must be a {ndim}-D {dtype} tensor")


def _check_cache(name, cache, q):
    _on_gpu(name, cache, q.device)
    if cache.ndim != 4:
        raise ValueError(f"{name} must be [blocks, block_size, kv_heads, head_dim]")
    if cache.dtype != q.dtype:
        raise ValueError(f"{name} dtype {cache.dtype} differs from the query dtype {q.dtype}")
    if cache.shape[-1] != q.shape[-1]:
        raise ValueError(f"{name} head_dim differs from the query head_dim")
    if cache.stride(-1) != 1:
        raise ValueError(f"{name} must have a contiguous head dimension")


def _attention_inputs(q, key_cache, value_cache, block_tables, context_lengths):
    if q.ndim != 3:
        raise ValueError("q must be [rows, q_heads, head_dim]")
    dtype_code(q.dtype)
    _on_gpu("q", q, q.device)
    _check_cache("key_cache", key_cache, q)
    _check_cache("value_cache", value_cache, q)
    if value_cache.shape != key_cache.shape:
        raise ValueError("key_cache and value_cache shapes differ")
    if q.shape[1] == 0 or q.shape[1] % key_cache.shape[2]:
        raise ValueError("query heads must be a positive multiple of KV heads")
    _check_int("block_tables", block_tables, torch.int32, 2, q.device)
    _check_int("context_lengths", context_lengths, torch.int32, 1, q.device)
    if block_tables.shape[1] and block_tables.stride(1) != 1:
        raise ValueError("block_tables rows must be contiguous")
    if not context_lengths.is_contiguous():
        context_lengths = context_lengths.contiguous()
    if q.stride(-1) != 1:
        q = q.contiguous()
    return q, context_lengths


def paged_attention(q, key_cache, value_cache, block_tables, context_lengths, window: int = 0):
    """Single-query paged attention; ``window`` > 0 keeps the last ``window`` keys."""
    if type(window) is not int or window < 0:
        raise ValueError("window must be a nonnegative integer")
    q, context_lengths = _attention_inputs(q, key_cache, value_cache, block_tables,
                                           context_lengths)
    rows = q.shape[0]
    if block_tables.shape[0] != rows or context_lengths.shape[0] != rows:
        raise ValueError("block_tables and context_lengths must have one row per query row")
    output = torch.empty_like(q)
    if rows == 0:
        return output
    lib = library()
    heads, head_dim = q.shape[1], q.shape[2]
    nbytes = lib.vrh_paged_decode_workspace_bytes(rows, heads, head_dim)
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    lib.check(
        lib.vrh_paged_decode(
            dtype_code(q.dtype), output.data_ptr(), q.data_ptr(), key_cache.data_ptr(),
            value_cache.data_ptr(), block_tables.data_ptr(), context_lengths.data_ptr(), rows,
            heads, key_cache.shape[2], head_dim, key_cache.shape[1], block_tables.shape[1],
            block_tables.stride(0), q.stride(0), q.stride(1), output.stride(0), output.stride(1),
            *key_cache.stride()[:3], *value_cache.stride()[:3], window, workspace.data_ptr(),
            nbytes, _stream(q),
        ),
        "vrh_paged_decode",
    )
    return output


def paged_attention_noalloc(q, key_cache, value_cache, block_tables, context_lengths,
                            window: int = 0, out=None):
    """``paged_attention`` without a workspace allocation: the split partials use
    the library's built-in per-GPU scratch (``vrh_paged_decode_noalloc``), and
    ``out`` may be given so that the call allocates nothing at all. Calls that
    overlap on one GPU share that scratch and race."""
    if type(window) is not int or window < 0:
        raise ValueError("window must be a nonnegative integer")
    q, context_lengths = _attention_inputs(q, key_cache, value_cache, block_tables,
                                           context_lengths)
    rows = q.shape[0]
    if block_tables.shape[0] != rows or context_lengths.shape[0] != rows:
        raise ValueError("block_tables and context_lengths must have one row per query row")
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or out.device != q.device \
            or out.stride(-1) != 1:
        raise ValueError("out must match q's shape, dtype and device, with a contiguous head_dim")
    if rows == 0:
        return out
    lib = library()
    lib.check(
        lib.vrh_paged_decode_noalloc(
            dtype_code(q.dtype), out.data_ptr(), q.data_ptr(), key_cache.data_ptr(),
            value_cache.data_ptr(), block_tables.data_ptr(), context_lengths.data_ptr(), rows,
            q.shape[1], key_cache.shape[2], q.shape[2], key_cache.shape[1], block_tables.shape[1],
            block_tables.stride(0), q.stride(0), q.stride(1), out.stride(0), out.stride(1),
            *key_cache.stride()[:3], *value_cache.stride()[:3], window, _stream(q),
        ),
        "vrh_paged_decode_noalloc",
    )
    return out


def paged_prefill_attention(q, key_cache, value_cache, block_tables, context_lengths,
                            cu_seqlens_q, max_seqlen_q):
    """Packed causal prefill, bottom-right aligned per sequence."""
    q, context_lengths = _attention_inputs(q, key_cache, value_cache, block_tables,
                                           context_lengths)
    _check_int("cu_seqlens_q", cu_seqlens_q, torch.int32, 1, q.device)
    sequences = block_tables.shape[0]
    if context_lengths.shape[0] != sequences or cu_seqlens_q.shape[0] != sequences + 1:
        raise ValueError("prefill metadata must describe the same number of sequences")
    output = torch.empty_like(q)
    if q.shape[0] == 0 or sequences == 0:
        return output
    cu_seqlens_q = cu_seqlens_q.contiguous()
    lib = library()
    nbytes = lib.vrh_paged_prefill_workspace_bytes(sequences, int(max_seqlen_q), q.shape[1],
                                                   q.shape[2])
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    lib.check(
        lib.vrh_paged_prefill(
            dtype_code(q.dtype), output.data_ptr(), q.data_ptr(), key_cache.data_ptr(),
            value_cache.data_ptr(), block_tables.data_ptr(), context_lengths.data_ptr(),
            cu_seqlens_q.data_ptr(), sequences, q.shape[0], int(max_seqlen_q), q.shape[1],
            key_cache.shape[2], q.shape[2], key_cache.shape[1], block_tables.shape[1],
            block_tables.stride(0), q.stride(0), q.stride(1), output.stride(0), output.stride(1),
            *key_cache.stride()[:3], *value_cache.stride()[:3], workspace.data_ptr(), nbytes,
            _stream(q),
        ),
        "vrh_paged_prefill",
    )
    return output


class HipPagedAttention:
    """gfx950 single-query decode, sliding-window decode and packed prefill."""

    def __call__(self, q, key_cache, value_cache, block_tables, context_lengths):
        return paged_attention(q, key_cache, value_cache, block_tables, context_lengths)

    def windowed(self, q, key_cache, value_cache, block_tables, context_lengths, window):
        if isinstance(window, bool) or not isinstance(window, int) or window <= 0:
            raise ValueError("window must be a positive integer")
        return paged_attention(q, key_cache, value_cache, block_tables, context_lengths,
                               window=window)

    def prefill(self, q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q,
                max_seqlen_q):
        return paged_prefill_attention(q, key_cache, value_cache, block_tables, context_lengths,
                                       cu_seqlens_q, max_seqlen_q)


# ----------------------------------------------------------------- KV writes
def _check_rows_tensor(name, tensor, rows, dtype, device):
    _check_int(name, tensor, dtype, 1, device)
    if tensor.shape[0] < rows:
        raise ValueError(f"{name} must have at least {rows} entries")


def kv_append(key_cache, value_cache, k, v, write_blocks, write_offsets, *, write_mask=None,
              active_rows=None):
    """Scatter ``k, v : [rows, kv_heads, head_dim]`` into one layer view.

    ``key_cache``/``value_cache`` are ``[blocks, block_size, kv_heads, head_dim]``
    views (e.g. ``cache[:, layer]``). Row r goes to
    ``[write_blocks[r], write_offsets[r]]`` unless ``write_mask[r]`` is false or
    ``r >= active_rows`` (a device int32 scalar). Bit-exact.
    """
    if key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("caches must be matching [blocks, block_size, kv_heads, head_dim] views")
    if key_cache.stride() != value_cache.stride():
        raise ValueError("key_cache and value_cache must share strides")
    return _append(key_cache, value_cache, k, v, write_blocks, write_offsets, write_mask,
                   active_rows, layers=1, cache_layer_stride=0)


def kv_append_layers(key_cache, value_cache, first_layer, k, v, write_blocks, write_offsets,
                     *, write_mask=None):
    """Append ``k, v : [layers, rows, kv_heads, head_dim]`` for consecutive layers
    ``first_layer ..`` of the full pool ``[blocks, layers, block_size, kv_heads, D]``
    in one launch (one step's appends of every layer)."""
    if key_cache.ndim != 5 or value_cache.shape != key_cache.shape:
        raise ValueError("caches must be matching 5-D pools")
    if key_cache.stride() != value_cache.stride():
        raise ValueError("key_cache and value_cache must share strides")
    if k.ndim != 4 or v.shape != k.shape:
        raise ValueError("k and v must be [layers, rows, kv_heads, head_dim]")
    layers = k.shape[0]
    if not 0 <= first_layer or first_layer + layers > key_cache.shape[1]:
        raise ValueError("layer range outside the pool")
    kview = key_cache[:, first_layer]
    vview = value_cache[:, first_layer]
    return _append(kview, vview, k, v, write_blocks, write_offsets, write_mask, None,
                   layers=layers, cache_layer_stride=key_cache.stride(1))


def _append(kc, vc, k, v, blocks, offsets, mask, active, *, layers, cache_layer_stride):
    dtype_code(kc.dtype)
    device = kc.device
    _on_gpu("key_cache", kc, device)
    _on_gpu("value_cache", vc, device)
    batched = layers > 1 or k.ndim == 4
    kk = k if batched else k.unsqueeze(0)
    vv = v if batched else v.unsqueeze(0)
    for name, tensor in (("k", kk), ("v", vv)):
        _on_gpu(name, tensor, device)
        if tensor.dtype != kc.dtype:
            raise ValueError(f"{name} must use the cache dtype {kc.dtype}")
        if tensor.shape[2:] != kc.shape[2:]:
            raise ValueError(f"{name} must be [rows, {kc.shape[2]}, {kc.shape[3]}]")
        if tensor.stride(-1) != 1:
            raise ValueError(f"{name} must have a contiguous head dimension")
    if kc.stride(-1) != 1:
        raise ValueError("caches must have a contiguous head dimension")
    rows = kk.shape[1]
    if vv.shape[1] != rows:
        raise ValueError("k and v must have the same rows")
    _check_rows_tensor("write_blocks", blocks, rows, torch.int64, device)
    _check_rows_tensor("write_offsets", offsets, rows, torch.int64, device)
    if mask is not None:
        _check_rows_tensor("write_mask", mask, rows, torch.bool, device)
    if active is not None:
        _on_gpu("active_rows", active, device)
        if active.dtype != torch.int32 or active.numel() != 1:
            raise ValueError("active_rows must be a device int32 scalar")
    if rows == 0:
        return
    blocks, offsets = blocks.contiguous(), offsets.contiguous()
    lib = library()
    lib.check(
        lib.vrh_kv_append(
            dtype_code(kc.dtype), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
            kc.stride(2), cache_layer_stride, kk.data_ptr(), vv.data_ptr(), kk.stride(1),
            kk.stride(2), kk.stride(0), vv.stride(1), vv.stride(2), vv.stride(0),
            blocks.data_ptr(), offsets.data_ptr(),
            None if mask is None else mask.contiguous().data_ptr(),
            None if active is None else active.data_ptr(), rows, layers, kc.shape[2],
            kc.shape[3], kc.shape[0], kc.shape[1], _stream(kc),
        ),
        "vrh_kv_append",
    )


# ------------------------------------------------------------ KV movement
def _slot_layout(cache, name):
    """Byte strides of a pool/layer view whose (kv_heads, head_dim) slot is dense."""
    if cache.stride(-1) != 1 or cache.stride(-2) != cache.shape[-1]:
        raise ValueError(f"{name} token slots must be contiguous [kv_heads, head_dim]")
    es = cache.element_size()
    return es, cache.shape[-2] * cache.shape[-1] * es


def kv_gather(key_cache, value_cache, table, length):
    """Materialise ``K[table[t // bs], t % bs]`` for ``t < length`` as ``[length, H, D]``
    (and V) from one layer view ``[blocks, block_size, kv_heads, head_dim]``."""
    _on_gpu("key_cache", key_cache, key_cache.device)
    _check_int("table", table, torch.int32, 1, key_cache.device)
    if key_cache.stride() != value_cache.stride() or key_cache.shape != value_cache.shape:
        raise ValueError("key_cache and value_cache must match")
    es, channel = _slot_layout(key_cache, "key_cache")
    length = int(length)
    block_size = key_cache.shape[1]
    if length < 0 or -(-length // block_size) > table.shape[0]:
        raise ValueError("length exceeds the table")
    keys = torch.empty((length, *key_cache.shape[2:]), dtype=key_cache.dtype,
                       device=key_cache.device)
    values = torch.empty_like(keys)
    if length == 0:
        return keys, values
    table = table.contiguous()
    lib = library()
    lib.check(
        lib.vrh_kv_gather(
            keys.data_ptr(), values.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
            table.data_ptr(), length, block_size, key_cache.stride(0) * es,
            key_cache.stride(1) * es, channel, _stream(key_cache),
        ),
        "vrh_kv_gather",
    )
    return keys, values


def kv_finalize(key_cache, value_cache, descriptors, tables, planes):
    """LAST_EXITED propagation of every layer for device rows (slot, depth, pos).

    ``tables`` is ``[slots * planes, width]`` int32; copies the exit plane's
    token slot into each deeper plane, as ``finalize_kernel`` does."""
    if key_cache.ndim != 5 or value_cache.shape != key_cache.shape:
        raise ValueError("caches must be matching 5-D pools")
    if key_cache.stride() != value_cache.stride():
        raise ValueError("key_cache and value_cache must share strides")
    device = key_cache.device
    _on_gpu("key_cache", key_cache, device)
    _check_int("descriptors", descriptors, torch.int64, 2, device)
    _check_int("tables", tables, torch.int32, 2, device)
    if descriptors.shape[1] != 3:
        raise ValueError("descriptors must be [rows, 3] (slot, depth, position)")
    es, channel = _slot_layout(key_cache, "key_cache")
    rows = descriptors.shape[0]
    if rows == 0 or planes <= 1:
        return
    descriptors, tables = descriptors.contiguous(), tables.contiguous()
    lib = library()
    lib.check(
        lib.vrh_kv_finalize(
            key_cache.data_ptr(), value_cache.data_ptr(), descriptors.data_ptr(),
            tables.data_ptr(), rows, planes, tables.shape[1], key_cache.shape[2],
            key_cache.shape[1], key_cache.stride(0) * es, key_cache.stride(1) * es,
            key_cache.stride(2) * es, channel, _stream(key_cache),
        ),
        "vrh_kv_finalize",
    )


def kv_finalize_token(key_cache, value_cache, src_block, dst_blocks, offset, layers):
    """Copy token slot ``offset`` of ``layers`` from block ``src_block`` into every
    block of ``dst_blocks`` (host integers: no host->device index tensor)."""
    import ctypes

    if key_cache.ndim != 5 or key_cache.stride() != value_cache.stride():
        raise ValueError("caches must be matching 5-D pools")
    es, channel = _slot_layout(key_cache, "key_cache")
    dst = (ctypes.c_int64 * max(1, len(dst_blocks)))(*[int(b) for b in dst_blocks])
    ids = (ctypes.c_int32 * max(1, len(layers)))(*[int(layer) for layer in layers])
    if not dst_blocks or not layers:
        return
    lib = library()
    lib.check(
        lib.vrh_kv_finalize_token(
            key_cache.data_ptr(), value_cache.data_ptr(), int(src_block), dst, len(dst_blocks),
            int(offset), ids, len(layers), key_cache.stride(0) * es, key_cache.stride(1) * es,
            key_cache.stride(2) * es, channel, _stream(key_cache),
        ),
        "vrh_kv_finalize_token",
    )


def kv_copy_blocks(key_cache, value_cache, src_blocks, dst_blocks):
    """``cache[dst_blocks[i]] = cache[src_blocks[i]]`` for whole blocks (all layers)
    of both pools; int64 device index tensors; disjoint source/destination sets."""
    device = key_cache.device
    _on_gpu("key_cache", key_cache, device)
    if key_cache.shape != value_cache.shape or key_cache.stride() != value_cache.stride():
        raise ValueError("key_cache and value_cache must match")
    _check_int("src_blocks", src_blocks, torch.int64, 1, device)
    _check_int("dst_blocks", dst_blocks, torch.int64, 1, device)
    if src_blocks.shape != dst_blocks.shape:
        raise ValueError("src_blocks and dst_blocks must have equal lengths")
    block = key_cache[0]
    if not block.is_contiguous():
        raise ValueError("each pool block must be contiguous")
    es = key_cache.element_size()
    n = src_blocks.shape[0]
    if n == 0:
        return
    src_blocks, dst_blocks = src_blocks.contiguous(), dst_blocks.contiguous()
    lib = library()
    lib.check(
        lib.vrh_kv_copy_blocks(
            key_cache.data_ptr(), value_cache.data_ptr(), key_cache.stride(0) * es,
            block.numel() * es, src_blocks.data_ptr(), dst_blocks.data_ptr(), n,
            _stream(key_cache),
        ),
        "vrh_kv_copy_blocks",
    )


def _offload_args(key_cache, value_cache, blocks, host_keys, host_values):
    device = key_cache.device
    _on_gpu("key_cache", key_cache, device)
    if key_cache.shape != value_cache.shape or key_cache.stride() != value_cache.stride():
        raise ValueError("key_cache and value_cache must match")
    _check_int("blocks", blocks, torch.int64, 1, device)
    block = key_cache[0]
    if not block.is_contiguous():
        raise ValueError("each pool block must be contiguous")
    shape = (blocks.shape[0], *key_cache.shape[1:])
    for name, host in (("host_keys", host_keys), ("host_values", host_values)):
        if host.device.type != "cpu" or not host.is_pinned():
            raise ValueError(f"{name} must be a pinned host tensor (pin_memory=True)")
        if tuple(host.shape) != shape or host.dtype != key_cache.dtype or not host.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {key_cache.dtype} tensor of shape "
                             f"{list(shape)}")
    es = key_cache.element_size()
    return key_cache.stride(0) * es, block.numel() * es


def kv_blocks_to_host(key_cache, value_cache, blocks, host_keys, host_values):
    """Row i of the pinned host tensors = block blocks[i] of each pool (all layers):
    the snapshot copies of core/kv_cache_manager.py:481-502 in one launch. The rows
    are complete once the current stream has passed this call."""
    stride, nbytes = _offload_args(key_cache, value_cache, blocks, host_keys, host_values)
    if blocks.shape[0] == 0:
        return
    lib = library()
    lib.check(
        lib.vrh_kv_blocks_to_host(
            key_cache.data_ptr(), value_cache.data_ptr(), stride, nbytes,
            blocks.contiguous().data_ptr(), host_keys.data_ptr(), host_values.data_ptr(),
            blocks.shape[0], _stream(key_cache),
        ),
        "vrh_kv_blocks_to_host",
    )


def kv_blocks_from_host(key_cache, value_cache, blocks, host_keys, host_values):
    """Block blocks[i] of each pool = row i of the pinned host tensors: the restore
    copies of core/kv_cache_manager.py:504-523 in one launch. The host rows must
    stay alive until the current stream has passed this call."""
    stride, nbytes = _offload_args(key_cache, value_cache, blocks, host_keys, host_values)
    if blocks.shape[0] == 0:
        return
    lib = library()
    lib.check(
        lib.vrh_kv_blocks_from_host(
            key_cache.data_ptr(), value_cache.data_ptr(), stride, nbytes,
            blocks.contiguous().data_ptr(), host_keys.data_ptr(), host_values.data_ptr(),
            blocks.shape[0], _stream(key_cache),
        ),
        "vrh_kv_blocks_from_host",
    )


# --------------------------------------------------------------- addresses
def expand_kv_addresses(positions, sequences, tables, page, blocks=None, offsets=None):
    """``blocks[i] = tables[sequences[i], positions[i] // page]``, ``offsets[i] =
    positions[i] % page``; int64 outputs (allocated when not given)."""
    device = positions.device
    _check_int("positions", positions, torch.int64, 1, device)
    _check_int("sequences", sequences, torch.int32, 1, device)
    _check_int("tables", tables, torch.int32, 2, device)
    n = positions.shape[0]
    if sequences.shape[0] < n:
        raise ValueError("sequences must cover every position")
    blocks = torch.empty(n, dtype=torch.int64, device=device) if blocks is None else blocks
    offsets = torch.empty(n, dtype=torch.int64, device=device) if offsets is None else offsets
    _check_rows_tensor("blocks", blocks, n, torch.int64, device)
    _check_rows_tensor("offsets", offsets, n, torch.int64, device)
    if n:
        tables = tables.contiguous()
        lib = library()
        lib.check(
            lib.vrh_expand_kv_addresses(
                positions.contiguous().data_ptr(), sequences.contiguous().data_ptr(),
                tables.data_ptr(), blocks.data_ptr(), offsets.data_ptr(), n, tables.shape[1],
                int(page), _stream(positions),
            ),
            "vrh_expand_kv_addresses",
        )
    return blocks, offsets


def routing_metadata(descriptors, tables, *, n, size, width, page, planes, out_width, slots,
                     positions, lengths, blocks, offsets, out_tables):
    """Device expansion of (slot, depth, pos) descriptors, as ``metadata_kernel``."""
    device = tables.device
    _check_int("descriptors", descriptors, torch.int64, 2, device)
    _check_int("tables", tables, torch.int32, 2, device)
    for name, tensor, dtype in (("slots", slots, torch.int64), ("positions", positions, torch.int64),
                                ("lengths", lengths, torch.int32), ("blocks", blocks, torch.int64),
                                ("offsets", offsets, torch.int64)):
        _check_rows_tensor(name, tensor, size, dtype, device)
    _check_int("out_tables", out_tables, torch.int32, 2, device)
    if out_tables.shape[0] < size or out_tables.stride(0) != width or not tables.is_contiguous():
        raise ValueError("out_tables must be [>= size, width] and tables contiguous")
    lib = library()
    lib.check(
        lib.vrh_routing_metadata(
            descriptors.data_ptr(), tables.data_ptr(), slots.data_ptr(), positions.data_ptr(),
            lengths.data_ptr(), blocks.data_ptr(), offsets.data_ptr(), out_tables.data_ptr(), n,
            size, width, page, planes, out_width, _stream(tables),
        ),
        "vrh_routing_metadata",
    )


def routing_slots(descriptors, slots, n, size):
    device = slots.device
    _check_int("descriptors", descriptors, torch.int64, 2, device)
    _check_rows_tensor("slots", slots, size, torch.int64, device)
    lib = library()
    lib.check(
        lib.vrh_routing_slots(descriptors.data_ptr(), slots.data_ptr(), n, size, _stream(slots)),
        "vrh_routing_slots",
    )
